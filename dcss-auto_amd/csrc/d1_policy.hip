// d1hip: rollout-side kernels that sit around the policy network on MI355X.
//   k_sample — categorical sampling with the Philox counter RNG (one lane per env).
//   k_gae    — reverse-time GAE scan (one lane per env, loop over T; each time step's
//              loads and stores are coalesced across envs), HBM-bound.
// Built with -ffp-contract=off: GAE products are rounded separately, as the
// reference's elementwise PyTorch ops are (gpu-d1/scripts/run_ring_ablations.py:354-360).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/d1hip.h"

namespace d1p {

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

__global__ __launch_bounds__(256) void k_sample(const float *__restrict__ logits, int n, int k, int ld, uint32_t key0,
                                                uint32_t key1, uint32_t t, int64_t *__restrict__ actions,
                                                float *__restrict__ logp) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float *l = logits + (size_t)i * ld;
    float m = l[0];
    for (int j = 1; j < k; j++) m = fmaxf(m, l[j]);
    float s = 0.f;
    for (int j = 0; j < k; j++) s += expf(l[j] - m);
    uint32_t w = philox_w0(0u, t, (uint32_t)i, 3u, key0, key1);
    float u = (float)(w >> 8) * (1.0f / 16777216.0f);
    float c = 0.f;
    int a = k - 1;
    for (int j = 0; j < k; j++) {
        c += expf(l[j] - m) / s;
        if (u < c) { a = j; break; }
    }
    if (actions) actions[i] = a;
    if (logp) logp[i] = l[a] - m - logf(s);
}

__global__ __launch_bounds__(256) void k_gae(const float *__restrict__ reward, const uint8_t *__restrict__ done,
                                             const float *__restrict__ value, const float *__restrict__ bootstrap,
                                             int T, int n, float gamma, float gl, float *__restrict__ adv,
                                             float *__restrict__ ret) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float next = bootstrap[i], gae = 0.f;
    for (int t = T - 1; t >= 0; t--) {
        size_t o = (size_t)t * n + i;
        float live = 1.f - (float)done[o];
        float v = value[o];
        float g1 = gamma * next;
        float g2 = g1 * live;
        float s = reward[o] + g2;
        float delta = s - v;
        float c = gl * live;
        float cg = c * gae;
        gae = delta + cg;
        adv[o] = gae;
        if (ret) ret[o] = gae + v;
        next = v;
    }
}

// uint8 -> bf16 widening of the observation batch (exact: every byte value has at most
// 8 significant bits). 16 bytes in, 32 bytes out per lane.
__global__ __launch_bounds__(256) void k_u8_bf16(const uint4 *__restrict__ in, uint4 *__restrict__ out, size_t n16) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n16) return;
    uint4 v = in[i];
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint32_t b0 = (w[j] >> (16 * h)) & 0xFFu, b1 = (w[j] >> (16 * h + 8)) & 0xFFu;
            o[2 * j + h] = (__float_as_uint((float)b0) >> 16) | (__float_as_uint((float)b1) & 0xFFFF0000u);
        }
    }
    out[2 * i] = make_uint4(o[0], o[1], o[2], o[3]);
    out[2 * i + 1] = make_uint4(o[4], o[5], o[6], o[7]);
}

}  // namespace d1p

extern "C" {
int d1_sample(const float *logits, int n, int k, int ld, uint64_t seed, uint32_t t, int64_t *actions, float *logp,
              void *stream) {
    if (n < 0 || k < 1 || k > 64 || ld < k || (n && !logits)) return D1_E_ARG;
    if (n == 0) return 0;
    hipLaunchKernelGGL(d1p::k_sample, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, logits, n, k, ld,
                       (uint32_t)seed, (uint32_t)(seed >> 32), t, actions, logp);
    return (int)hipGetLastError();
}
int d1_obs_to_bf16(const uint8_t *obs, void *out, int64_t count, void *stream) {
    if (count < 0 || (count % 16) || (count && (!obs || !out))) return D1_E_ARG;
    if (((uintptr_t)obs & 15) || ((uintptr_t)out & 15)) return D1_E_ARG;
    if (count == 0) return 0;
    size_t n16 = (size_t)count / 16;
    hipLaunchKernelGGL(d1p::k_u8_bf16, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint4 *)obs, (uint4 *)out, n16);
    return (int)hipGetLastError();
}
int d1_gae(const float *reward, const uint8_t *done, const float *value, const float *bootstrap, int T, int n,
           float gamma, float gamma_lambda, float *adv, float *returns, void *stream) {
    if (T < 0 || n < 0 || ((T && n) && (!reward || !done || !value || !bootstrap || !adv))) return D1_E_ARG;
    if (T == 0 || n == 0) return 0;
    hipLaunchKernelGGL(d1p::k_gae, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, reward, done, value,
                       bootstrap, T, n, gamma, gamma_lambda, adv, returns);
    return (int)hipGetLastError();
}
}
