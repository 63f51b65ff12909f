/* Helpers shared between the oracle's translation units -- TEST INFRASTRUCTURE ONLY. */
#ifndef LAYA_ORACLE_INTERNAL_H
#define LAYA_ORACLE_INTERNAL_H

/* Runs f(ctx, lo, hi) over [0, n) split into contiguous ranges on `workers` threads. */
void or_parallel(int n, int workers, void (*f)(void *, int, int), void *ctx);

#endif
