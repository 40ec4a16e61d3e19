/*
 * cpu_baseline.c -- row-parallel driver over the oracle's MatMulRows.
 *
 * TEST INFRASTRUCTURE ONLY (the timed CPU baseline of bench.py).  The work
 * split follows MatMulBatch.RunShard (src/Needle/Quant.cs:710-723): rows in
 * blocks of Quant.RowBlock = 4, member m of M takes blocks
 * [m*B/M, (m+1)*B/M).  Workers are a persistent spin pool, as
 * src/Needle/Pool.cs keeps its team spinning between calls.  Every member
 * runs or_matmul_rows_i8 on its rows, so results are bit-identical to the
 * single-threaded oracle; or_baseline_simd_matmul_i8 runs the SIMD tier
 * (cpu_simd.c) on each member's rows instead.
 */
#define _GNU_SOURCE
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdlib.h>

#include "needle_oracle.h"

typedef struct {
    int tier; /* OR_TIER_SCALAR: or_matmul_rows_i8, else or_simd_matmul_i8 */
    const int8_t* w;
    const uint16_t* scales;
    int rows, cols, group;
    const int8_t* q;
    const float* qscale;
    int tokens;
    float* y;
    int ldy, row_start, row_end;
} job_t;

static struct {
    int members;
    pthread_t threads[256];
    atomic_int generation;
    atomic_int done;
    atomic_int stop;
    job_t job;
} pool;

static void run_member(int m)
{
    const job_t* j = &pool.job;
    int blocks = (j->row_end - j->row_start + 3) / 4;
    int first = (int)((long)m * blocks / pool.members);
    int end = (int)((long)(m + 1) * blocks / pool.members);
    int r0 = j->row_start + first * 4;
    int r1 = j->row_start + end * 4;
    if (r1 > j->row_end) r1 = j->row_end;
    if (r0 < r1 && j->tier != OR_TIER_SCALAR)
        or_simd_matmul_i8(j->tier, j->w, j->scales, j->rows, j->cols, j->q, j->qscale, j->tokens, j->y, j->ldy, r0,
                          r1);
    else if (r0 < r1)
        or_matmul_rows_i8(j->w, j->scales, j->rows, j->cols, j->group, j->q, j->qscale, j->tokens, j->y, j->ldy,
                          r0, r1);
}

static void* worker(void* arg)
{
    int m = (int)(long)arg;
    int seen = 0;
    for (;;) {
        int g;
        while ((g = atomic_load_explicit(&pool.generation, memory_order_acquire)) == seen) {
            if (atomic_load(&pool.stop)) return NULL;
            sched_yield();
        }
        seen = g;
        run_member(m);
        atomic_fetch_add_explicit(&pool.done, 1, memory_order_release);
    }
}

/* Starts (or resizes) the pool; returns the member count in use. */
int or_baseline_start(int members)
{
    if (members < 1) members = 1;
    if (members > 256) members = 256;
    if (pool.members == members) return members;
    if (pool.members > 0) {
        atomic_store(&pool.stop, 1);
        for (int i = 1; i < pool.members; i++) pthread_join(pool.threads[i], NULL);
        atomic_store(&pool.stop, 0);
    }
    pool.members = members;
    atomic_store(&pool.generation, 0);
    for (int i = 1; i < members; i++) pthread_create(&pool.threads[i], NULL, worker, (void*)(long)i);
    return members;
}

void or_baseline_stop(void)
{
    if (pool.members > 0) {
        atomic_store(&pool.stop, 1);
        for (int i = 1; i < pool.members; i++) pthread_join(pool.threads[i], NULL);
        atomic_store(&pool.stop, 0);
        pool.members = 0;
    }
}

static void run_pool(const job_t* j)
{
    pool.job = *j;
    atomic_store(&pool.done, 0);
    atomic_fetch_add_explicit(&pool.generation, 1, memory_order_release);
    run_member(0);
    while (atomic_load_explicit(&pool.done, memory_order_acquire) < pool.members - 1) sched_yield();
}

void or_baseline_matmul_i8(const int8_t* w, const uint16_t* scales, int rows, int cols, int group, const int8_t* q,
                           const float* qscale, int tokens, float* y, int ldy, int row_start, int row_end)
{
    if (pool.members <= 1) {
        or_matmul_rows_i8(w, scales, rows, cols, group, q, qscale, tokens, y, ldy, row_start, row_end);
        return;
    }
    job_t j = {OR_TIER_SCALAR, w, scales, rows, cols, group, q, qscale, tokens, y, ldy, row_start, row_end};
    run_pool(&j);
}

void or_baseline_simd_matmul_i8(int tier, const int8_t* w, const uint16_t* scales, int rows, int cols,
                                const int8_t* q, const float* qscale, int tokens, float* y, int ldy, int row_start,
                                int row_end)
{
    if (pool.members <= 1) {
        or_simd_matmul_i8(tier, w, scales, rows, cols, q, qscale, tokens, y, ldy, row_start, row_end);
        return;
    }
    job_t j = {tier, w, scales, rows, cols, 32, q, qscale, tokens, y, ldy, row_start, row_end};
    run_pool(&j);
}
