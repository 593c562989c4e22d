/* orc_bigmat.c -- seeded inputs, carry normalisation and comparison.
 * Test infrastructure only (see oracle.h). */
#include <stdlib.h>
#include <string.h>
#include "oracle.h"

/* SplitMix64 (Steele, Lea, Flood 2014; the constants are the published
 * ones).  Follows src/bigmat.c:21-27: the state advances by the golden gamma
 * before mixing, so output i (0-based) is mix(seed + (i+1)*gamma). */
uint64_t orc_sm64_next(uint64_t *state)
{
    *state += 0x9E3779B97F4A7C15ULL;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* src/bigmat.c:29-35: limbs in plane-major index order, low 16 bits of
 * successive outputs. */
void orc_bigmat_rand(uint16_t *m, int n, int L, uint64_t seed)
{
    uint64_t s = seed;
    size_t total = (size_t)n * n * (size_t)L;
    for (size_t i = 0; i < total; i++)
        m[i] = (uint16_t)orc_sm64_next(&s);
}

/* src/bigmat.c:37-46 */
void orc_to_entry_major(const uint16_t *plane, int n, int L, uint16_t *em)
{
    size_t nn = (size_t)n * n;
    for (int u = 0; u < L; u++)
        for (size_t e = 0; e < nn; e++)
            em[e * L + u] = plane[(size_t)u * nn + e];
}

/* src/bigmat.c:48-60: per element, ascending limb index, arithmetic shift
 * for the carry, so signed accumulators give two's complement mod
 * 2^(16*RL). */
void orc_normalize_planes(const int64_t *acc, int nplanes, int n,
                          uint16_t *out, int RL)
{
    size_t nn = (size_t)n * n;
    for (size_t e = 0; e < nn; e++) {
        int64_t carry = 0;
        for (int w = 0; w < RL; w++) {
            int64_t v = carry + (w < nplanes ? acc[(size_t)w * nn + e] : 0);
            out[(size_t)w * nn + e] = (uint16_t)(v & 0xFFFF);
            carry = v >> ORC_LIMB_BITS;
        }
    }
}

/* src/bigmat.c:62-75: first mismatch in plane order. */
int orc_bigres_equal(const uint16_t *a, const uint16_t *b, int n, int RL,
                     int *bad_i, int *bad_j, int *bad_w)
{
    size_t nn = (size_t)n * n;
    for (int w = 0; w < RL; w++) {
        const uint16_t *pa = a + (size_t)w * nn, *pb = b + (size_t)w * nn;
        for (size_t e = 0; e < nn; e++)
            if (pa[e] != pb[e]) {
                if (bad_w) *bad_w = w;
                if (bad_i) *bad_i = (int)(e / (size_t)n);
                if (bad_j) *bad_j = (int)(e % (size_t)n);
                return 0;
            }
    }
    return 1;
}
