/*
 * expf_check.c -- runs the device expf restatement (qwen.haiku_amd/csrc/
 * qk_expf.h, compiled here as plain C) against the host libm expf on
 * every stride-th float bit pattern, on 8 threads. Prints the mismatch
 * count and the first mismatching input. Test infrastructure for
 * tests/test_oracle.py.
 *
 * usage: expf_check STRIDE
 */
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>

#include "qk_expf.h"

#define THREADS 8

static uint64_t stride;
static unsigned long long bad[THREADS];
static uint32_t first[THREADS];

static uint32_t bits32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static void *run(void *p) {
    const int id = (int)(long)p;
    for (uint64_t u = (uint64_t)id * stride; u < (1ULL << 32); u += THREADS * stride) {
        const uint32_t b = (uint32_t)u;
        float x;
        memcpy(&x, &b, 4);
        const float want = expf(x), got = qk_expf(x);
        if (bits32(want) != bits32(got) && !(want != want && got != got)) {
            if (!bad[id] || b < first[id]) first[id] = b;
            bad[id]++;
        }
    }
    return NULL;
}

int main(int argc, char **argv) {
    stride = argc > 1 ? strtoull(argv[1], NULL, 0) : 1;
    if (stride < 1) stride = 1;
    pthread_t th[THREADS];
    for (long i = 0; i < THREADS; i++) pthread_create(&th[i], NULL, run, (void *)i);
    unsigned long long total = 0;
    uint32_t f = 0xffffffffu;
    for (int i = 0; i < THREADS; i++) {
        pthread_join(th[i], NULL);
        total += bad[i];
        if (bad[i] && first[i] < f) f = first[i];
    }
    printf("%llu %08x\n", total, f);
    return 0;
}
