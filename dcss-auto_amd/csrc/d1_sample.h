// d1hip: the categorical sampler's per-row arithmetic, shared by the standalone sampler
// (d1_policy.hip) and the policy forward's fused epilogue (d1_forward.hip) so that both
// give bit-identical actions and log-probabilities. Both files are built with
// -ffp-contract=off.
//
// Row i at counter step t: u = (w >> 8) * 2^-24 with w = word 0 of
// Philox4x32-10(ctr = {0, t, i, 3}, key = {key0, key1}) (Salmon et al., SC'11: multipliers
// 0xD2511F53 / 0xCD9E8D57, Weyl increments 0x9E3779B9 / 0xBB67AE85); the action is the
// first j with u < sum_{j' <= j} exp(l_j' - max) / sum exp(l - max) (fp32, left to right),
// else k - 1; log p = l_a - max - log(sum).
#ifndef D1_SAMPLE_H
#define D1_SAMPLE_H
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace d1s {

__device__ inline uint32_t philox_w0(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; r++) {
        uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
        uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
        uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
        k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
    }
    return c0;
}

// words 0 and 1 of the same Philox4x32-10 block (the two uniforms of the two-stage sample)
__device__ inline void philox_w01(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0, uint32_t k1,
                                  uint32_t &w0, uint32_t &w1) {
#pragma unroll
    for (int r = 0; r < 10; r++) {
        uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
        uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
        uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
        k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
    }
    w0 = c0;
    w1 = c1;
}
__device__ __forceinline__ float unit24(uint32_t w) { return (float)(w >> 8) * (1.0f / 16777216.0f); }

// Inverse-CDF draw of one categorical row with uniform u: the first j with u < the running
// sum of exp(l_j - max) / sum exp(l - max) (fp32, left to right), else k - 1; log p =
// l_a - max - log(sum). The running sum keeps going past the choice and l_a is kept as the
// loop passes it, which changes nothing: with a constant k (register-held rows) the loops
// unroll completely and no row element is indexed at run time.
template <class L>
__device__ __forceinline__ void cat_core(L l, int k, float u, int &a, float &lp) {
    float m = l(0);
#pragma unroll
    for (int j = 1; j < k; j++) m = fmaxf(m, l(j));
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < k; j++) s += expf(l(j) - m);
    float c = 0.f, la = l(k - 1);
    bool found = false;
    a = k - 1;
#pragma unroll
    for (int j = 0; j < k; j++) {
        const float lj = l(j);
        c += expf(lj - m) / s;
        if (!found && u < c) { a = j; la = lj; found = true; }
    }
    lp = la - m - logf(s);
}

// Env action of an autoregressive (verb, target) pair: verb 0 MOVE / 1 ATTACK with target
// (dx, dy) = (t % 5 - 2, t / 5 - 2) on the Chebyshev-1 ring -> direction d (N, E, S, W, NE,
// SE, SW, NW) -> d or 8 + d, other targets -> -1 (one WAIT turn); verb 2 WAIT (16), 3 REST
// (17), 4 DESCEND (18), 5-7 WAIT.
__device__ __forceinline__ int ar_action(int v, int tg) {
    if (v <= 1) {
        const int dx = tg % 5 - 2, dy = tg / 5 - 2;
        int d = -1;
        if (dx == 0 && dy == -1) d = 0; else if (dx == 1 && dy == 0) d = 1; else if (dx == 0 && dy == 1) d = 2;
        else if (dx == -1 && dy == 0) d = 3; else if (dx == 1 && dy == -1) d = 4; else if (dx == 1 && dy == 1) d = 5;
        else if (dx == -1 && dy == 1) d = 6; else if (dx == -1 && dy == -1) d = 7;
        return d < 0 ? -1 : d + 8 * v;
    }
    return v <= 4 ? 14 + v : 16;
}

// l(j) returns logit j of the row (global memory or registers)
template <class L>
__device__ __forceinline__ void sample_core(L l, int k, uint32_t key0, uint32_t key1, uint32_t t, uint32_t i, int &a,
                                            float &lp) {
    float m = l(0);
    for (int j = 1; j < k; j++) m = fmaxf(m, l(j));
    float s = 0.f;
    for (int j = 0; j < k; j++) s += expf(l(j) - m);
    const uint32_t w = philox_w0(0u, t, i, 3u, key0, key1);
    const float u = (float)(w >> 8) * (1.0f / 16777216.0f);
    float c = 0.f;
    a = k - 1;
    for (int j = 0; j < k; j++) {
        c += expf(l(j) - m) / s;
        if (u < c) { a = j; break; }
    }
    lp = l(a) - m - logf(s);
}

}  // namespace d1s
#endif
