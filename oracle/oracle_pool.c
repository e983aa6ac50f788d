/*
 * TEST INFRASTRUCTURE: the threading of the reference's thread_pool.c for
 * the oracle when it serves as the CPU baseline (bench.py's cpu_baseline
 * leg).  A persistent pool of spinning workers (thread_pool.c:110-137,
 * 208-238), and the reference's rule for how many run an operation: one
 * below 2*m*k*n = 16 Mi flops, every pool thread above (pick_nthreads,
 * thread_pool.c:25,178-185); work split into contiguous chunks of
 * ceil(n / nt) (matmul.c:107-114, nn.c:455-458).  The pool size is the
 * caller's (the physical cores the process may use).  Off by default:
 * then every operation runs on the calling thread.  The threading never
 * changes a result bit: every output element is one thread's complete dot.
 */
#define _GNU_SOURCE
#include "oracle_pool.h"

#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>

#define MIN_FLOPS_THREADED (16 * 1024 * 1024) /* thread_pool.c:25 */
#define MAX_POOL 256

static struct {
	int n;
	pthread_t th[MAX_POOL];
	atomic_int generation, n_done, quit;
	orc_task_fn fn;
	void *arg;
	int active;
} P;

static void *worker(void *p)
{
	const int idx = (int)(intptr_t)p;
	int gen = 0;
	for (;;) {
		/* spin as thread_pool.c:123-125 does, yielding after a while so an
		 * oversubscribed host still makes progress */
		for (int spin = 0; atomic_load_explicit(&P.generation, memory_order_acquire) == gen;
		     spin++) {
			if (spin < 20000)
				__builtin_ia32_pause();
			else
				sched_yield();
		}
		gen++;
		if (atomic_load(&P.quit))
			return NULL;
		if (idx < P.active)
			P.fn(P.arg, idx, P.active);
		atomic_fetch_add_explicit(&P.n_done, 1, memory_order_release);
	}
}

int orc_set_pool(int nthreads)
{
	if (P.n > 0) { /* stop the old pool */
		atomic_store(&P.quit, 1);
		atomic_fetch_add_explicit(&P.generation, 1, memory_order_release);
		for (int i = 0; i < P.n - 1; i++)
			pthread_join(P.th[i], NULL);
		P.n = 0;
	}
	atomic_store(&P.quit, 0);
	atomic_store(&P.generation, 0);
	if (nthreads <= 1)
		return 0;
	if (nthreads > MAX_POOL)
		nthreads = MAX_POOL;
	/* the calling thread is worker n - 1 */
	for (int i = 0; i < nthreads - 1; i++)
		if (pthread_create(&P.th[i], NULL, worker, (void *)(intptr_t)i) != 0) {
			P.n = i + 1;
			orc_set_pool(0);
			return -1;
		}
	P.n = nthreads;
	return nthreads;
}

int orc_pool_active(void)
{
	return P.n > 1;
}

int orc_pool_threads(size_t m, size_t k, size_t n)
{
	if (P.n <= 1 || 2 * m * k * n < MIN_FLOPS_THREADED)
		return 1;
	return P.n;
}

void orc_pool_run(orc_task_fn fn, void *arg, int nt)
{
	if (nt <= 1 || P.n <= 1) {
		fn(arg, 0, 1);
		return;
	}
	if (nt > P.n)
		nt = P.n;
	P.fn = fn;
	P.arg = arg;
	P.active = nt;
	atomic_store_explicit(&P.n_done, 0, memory_order_release);
	atomic_fetch_add_explicit(&P.generation, 1, memory_order_release);
	fn(arg, nt - 1, nt); /* the calling thread takes the last chunk */
	while (atomic_load_explicit(&P.n_done, memory_order_acquire) < P.n - 1)
		__builtin_ia32_pause();
}
