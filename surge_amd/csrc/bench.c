/* bench.c - decode-throughput yardsticks over a cumulative wall-time series
 * (reference surge.h:1784-1824, src/bench.c:23-78).
 *
 * t[i] is the wall time at which token i finished. Both estimators ignore
 * indices below `warmup`. The slope is a least-squares fit of token index
 * against time, done mean-centred in double so epoch-sized timestamps do not
 * cancel; the average is endpoint to endpoint. */
#include "surge.h"

double sg_bench_slope(const double *t, uint32_t n, uint32_t warmup) {
    if (!t || n <= warmup || n - warmup < 2) return 0.0;
    uint32_t k = n - warmup;
    double mt = 0.0, mi = 0.0;
    for (uint32_t i = warmup; i < n; i++) { mt += t[i]; mi += (double)i; }
    mt /= k; mi /= k;
    double sxy = 0.0, sxx = 0.0;
    for (uint32_t i = warmup; i < n; i++) {
        double dx = t[i] - mt;
        sxy += dx * ((double)i - mi);
        sxx += dx * dx;
    }
    return sxx > 0.0 ? sxy / sxx : 0.0;
}

double sg_bench_avg_tps(const double *t, uint32_t n, uint32_t warmup) {
    if (!t || n == 0 || warmup + 1 >= n) return 0.0;
    double dt = t[n - 1] - t[warmup];
    return dt > 0.0 ? (double)(n - 1 - warmup) / dt : 0.0;
}

uint32_t sg_bench_default_warmup(uint32_t n_gen) {
    uint32_t w = (uint32_t)(0.02 * (double)n_gen + 0.5);
    return w < 1 ? 1 : w;
}
