/* greedy.c - the argmax every greedy driver uses (reference surge.h:1503-1512,
 * src/greedy.c:17-27): scan upward, strict '>', so the lowest index wins an
 * exact tie. 0 for a NULL vector or n == 0. */
#include "surge.h"

uint32_t sg_argmax_f32(const float *v, uint32_t n) {
    if (!v || !n) return 0;
    uint32_t best = 0;
    float bv = v[0];
    for (uint32_t i = 1; i < n; i++)
        if (v[i] > bv) { bv = v[i]; best = i; }
    return best;
}
