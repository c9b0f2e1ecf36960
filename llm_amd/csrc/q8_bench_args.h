/*
 * q8_bench_args.h -- the argument block of the measurement kernels
 * (q8_probe.hip), shared with their host launcher (q8_bench.cpp).  Bench-only:
 * nothing of the product library (libq8mi.so) uses it.
 */
#ifndef Q8_BENCH_ARGS_H
#define Q8_BENCH_ARGS_H

#include <stdint.h>

typedef struct {
    int iters;          /* compute probes: loop trips per wave */
    int mask;           /* split probes: bit 0 runs waves 0-3 (role A), bit 1 waves 4-7 (role B) */
    unsigned never;     /* a value no result takes: results feed `sink` only when equal to it */
    unsigned *sink;
} Q8ProbeArgs;

#endif
