/* bm_microbench.c -- latency of the BlockManager operations through the C ABI,
 * on the same cases as the reference's criterion benches
 * (benches/block_manager.rs:35-134): a 4096-block pool of 16-token blocks, the
 * timed operations in batches of 256 with their setup untimed.
 *
 *   gcc -O2 -Iinclude tests/native/bm_microbench.c -Lzealot_amd -lzealot_kv \
 *       -Wl,-rpath,$PWD/zealot_amd -o bm_microbench && ./bm_microbench [rounds]
 *
 * Prints one line per case: name and nanoseconds per operation (the median
 * over the rounds of the mean of one batch). */
#include <stdio.h>
#include <stdlib.h>
#include <time.h>

#include "zealot_kv.h"

enum { POOL = 4096, BLOCK_SIZE = 16, BATCH = 256 };

static double now_ns(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec * 1e9 + (double)t.tv_nsec;
}

static int cmp(const void *a, const void *b) {
    const double x = *(const double *)a, y = *(const double *)b;
    return (x > y) - (x < y);
}

static double median(double *v, int n) {
    qsort(v, (size_t)n, sizeof(double), cmp);
    return v[n / 2];
}

static void must(int rc, const char *what) {
    if (rc != ZK_OK) {
        fprintf(stderr, "%s failed: %d (%s)\n", what, rc, zk_last_error());
        exit(1);
    }
}

int main(int argc, char **argv) {
    const int rounds = argc > 1 ? atoi(argv[1]) : 2000;
    double *t = malloc(sizeof(double) * (size_t)rounds);
    zk_block_handle h[BATCH];
    zk_block_manager *bm;
    volatile uint64_t sink = 0;

    /* allocate from a non-empty pool; the frees between batches are untimed */
    must(zk_bm_create(POOL, BLOCK_SIZE, &bm), "create");
    for (int r = 0; r < rounds; ++r) {
        const double t0 = now_ns();
        for (int i = 0; i < BATCH; ++i) {
            zk_bm_allocate(bm, &h[i]);
            sink += h[i].block_id;
        }
        t[r] = (now_ns() - t0) / BATCH;
        for (int i = 0; i < BATCH; ++i) must(zk_bm_free(bm, h[i]), "free");
    }
    printf("bm_allocate_1 %.1f\n", median(t, rounds));

    /* free that returns the block to the pool; the allocations are untimed */
    for (int r = 0; r < rounds; ++r) {
        for (int i = 0; i < BATCH; ++i) must(zk_bm_allocate(bm, &h[i]), "allocate");
        const double t0 = now_ns();
        for (int i = 0; i < BATCH; ++i) sink += (uint64_t)zk_bm_free(bm, h[i]);
        t[r] = (now_ns() - t0) / BATCH;
    }
    printf("bm_free_last_ref %.1f\n", median(t, rounds));

    /* reference of a live block */
    must(zk_bm_allocate(bm, &h[0]), "allocate");
    for (int r = 0; r < rounds; ++r) {
        const double t0 = now_ns();
        for (int i = 0; i < BATCH; ++i) sink += (uint64_t)zk_bm_reference(bm, h[0]);
        t[r] = (now_ns() - t0) / BATCH;
    }
    printf("bm_reference %.1f\n", median(t, rounds));

    /* a stale handle is rejected */
    zk_bm_destroy(bm);
    must(zk_bm_create(POOL, BLOCK_SIZE, &bm), "create");
    zk_block_handle stale;
    must(zk_bm_allocate(bm, &stale), "allocate");
    must(zk_bm_free(bm, stale), "free");
    for (int r = 0; r < rounds; ++r) {
        const double t0 = now_ns();
        for (int i = 0; i < BATCH; ++i) sink += (uint64_t)(zk_bm_free(bm, stale) != ZK_OK);
        t[r] = (now_ns() - t0) / BATCH;
    }
    printf("bm_stale_handle %.1f\n", median(t, rounds));

    /* allocation from an empty pool (OutOfBlocks) */
    zk_bm_destroy(bm);
    must(zk_bm_create(POOL, BLOCK_SIZE, &bm), "create");
    for (int i = 0; i < POOL; ++i) must(zk_bm_allocate(bm, &stale), "allocate");
    for (int r = 0; r < rounds; ++r) {
        const double t0 = now_ns();
        for (int i = 0; i < BATCH; ++i) sink += (uint64_t)(zk_bm_allocate(bm, &h[0]) != ZK_OK);
        t[r] = (now_ns() - t0) / BATCH;
    }
    printf("bm_allocate_full %.1f\n", median(t, rounds));

    zk_bm_destroy(bm);
    free(t);
    (void)sink;
    return 0;
}
