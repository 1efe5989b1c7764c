/*
 * C restatement of CRESSO5's coordinate hash (TEST INFRASTRUCTURE ONLY).
 *
 * Follows /root/reference/cresso_v5.py:495-516 (_hash_index_tensor): for the
 * row-major linear index i of an element and salt s' = salt + 1,
 *   h = i*(1103515245 + 97 s') + (12345 + 0x9E3779B1 s')
 *   h ^= h >> 16;  h *= 2246822519 + 1315423911 s'
 *   h ^= h >> 13;  h *= 3266489917 + 374761393 s'
 *   h ^= h >> 16;  bin = floor_mod(h, bins)
 * in int64 with two's-complement wrap and arithmetic right shifts.  Here the
 * wrap is done in uint64 (defined behaviour) and the arithmetic shift is
 * spelled out, so the result does not depend on implementation-defined C.
 * Used by tests to cross-check the numpy restatement and the HIP kernels.
 */
#include <stdint.h>

static int64_t wrap(uint64_t u) { return (int64_t)u; }

static uint64_t ashr(uint64_t x, unsigned k) {
    uint64_t r = x >> k;
    if (x >> 63) r |= ~(UINT64_MAX >> k);
    return r;
}

int64_t cresso_oracle_hash_bin(int64_t i, int64_t bins, int64_t salt) {
    uint64_t s = (uint64_t)(salt + 1);
    uint64_t h = (uint64_t)i * (1103515245ULL + 97ULL * s) + (12345ULL + 0x9E3779B1ULL * s);
    h ^= ashr(h, 16);
    h *= 2246822519ULL + 1315423911ULL * s;
    h ^= ashr(h, 13);
    h *= 3266489917ULL + 374761393ULL * s;
    h ^= ashr(h, 16);
    int64_t v = wrap(h);
    int64_t r = v % bins;
    if (r < 0) r += bins;
    return r;
}

void cresso_oracle_hash_bins(int64_t n, int64_t bins, int64_t salt, int32_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = (int32_t)cresso_oracle_hash_bin(i, bins, salt);
}

void cresso_oracle_hash_counts(int64_t n, int64_t bins, int64_t salt, int64_t* counts) {
    for (int64_t b = 0; b < bins; ++b) counts[b] = 0;
    for (int64_t i = 0; i < n; ++i) counts[cresso_oracle_hash_bin(i, bins, salt)] += 1;
}
