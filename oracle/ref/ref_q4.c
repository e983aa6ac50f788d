/*
 * TEST INFRASTRUCTURE: exposes the reference's only Q4_0 quantizer, the
 * static quantize_q4_0_block of test/quant.c:45-79 (the test file is
 * #included from the reference tree at build time; its main is renamed).
 */
#define main ref_quant_test_main
#include "test/quant.c"
#undef main

void ref_quantize_q4_0(const float *x, void *blocks, size_t n)
{
	block_q4_0 *b = blocks;
	for (size_t i = 0; i < n / GGML_QK; i++)
		quantize_q4_0_block(&x[i * GGML_QK], &b[i]);
}
