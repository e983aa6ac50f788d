/* TEST INFRASTRUCTURE: the oracle's copy of the reference's threading
 * (thread_pool.c), used when the oracle is timed as the CPU baseline. */
#ifndef ORACLE_POOL_H
#define ORACLE_POOL_H

#include <stddef.h>

typedef void (*orc_task_fn)(void *arg, int tidx, int nthreads);

/* threads an operation of 2*m*k*n flops runs on: 1 below 16 Mi or with
 * the pool off, else the pool size (pick_nthreads, thread_pool.c:178-185) */
int orc_pool_threads(size_t m, size_t k, size_t n);
/* 1 while a pool of two or more threads is set */
int orc_pool_active(void);
/* run fn(arg, i, nt) for i < nt on the pool, the caller taking i = nt - 1 */
void orc_pool_run(orc_task_fn fn, void *arg, int nt);

#endif
