// d1hip: rollout-side kernels that sit around the policy network on MI355X.
//   k_sample — categorical sampling with the Philox counter RNG (one lane per env).
//   k_gae    — reverse-time GAE scan (one lane per env, loop over T; each time step's
//              loads and stores are coalesced across envs), HBM-bound.
// Built with -ffp-contract=off: GAE products are rounded separately, as the
// reference's elementwise PyTorch ops are (gpu-d1/scripts/run_ring_ablations.py:354-360).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/d1hip.h"
#include "d1_sample.h"

namespace d1p {

using d1s::philox_w0;

// the sample of row i at counter step t (shared with the fused forward: identical results)
__device__ __forceinline__ void sample_row(const float *__restrict__ logits, int i, int k, int ld, uint32_t key0,
                                           uint32_t key1, uint32_t t, int64_t *__restrict__ actions,
                                           float *__restrict__ logp) {
    const float *l = logits + (size_t)i * ld;
    int a;
    float lp;
    d1s::sample_core([&](int j) { return l[j]; }, k, key0, key1, t, (uint32_t)i, a, lp);
    if (actions) actions[i] = a;
    if (logp) logp[i] = lp;
}

__global__ __launch_bounds__(256) void k_sample(const float *__restrict__ logits, int n, int k, int ld, uint32_t key0,
                                                uint32_t key1, uint32_t t, int64_t *__restrict__ actions,
                                                float *__restrict__ logp) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    sample_row(logits, i, k, ld, key0, key1, t, actions, logp);
}
// the counter step read from device memory (*t_dev + t_add), so that a captured graph
// samples a new step on every replay
__global__ __launch_bounds__(256) void k_sample_dev(const float *__restrict__ logits, int n, int k, int ld,
                                                    uint32_t key0, uint32_t key1, const uint32_t *__restrict__ t_dev,
                                                    uint32_t t_add, int64_t *__restrict__ actions,
                                                    float *__restrict__ logp) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    sample_row(logits, i, k, ld, key0, key1, *t_dev + t_add, actions, logp);
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

// Two-stage (autoregressive) sample: verb ~ softmax(verb_logits[i]) with u0, then
// target ~ softmax(target_logits[i][verb]) with u1, where u0/u1 = words 0/1 of
// Philox4x32-10(ctr={0, t, i, 3}, key) scaled to [0,1) with 24 bits (d1_sample.h, shared
// with the fused forward's epilogue); logp = log p(verb) + log p(target | verb); the env
// action is d1s::ar_action(verb, target).
__global__ __launch_bounds__(256) void k_sample_ar(const float *__restrict__ verb_logits, int nv, int ldv,
                                                   const float *__restrict__ target_logits, int nt, int ldt, int n,
                                                   uint32_t key0, uint32_t key1, uint32_t t, int32_t *__restrict__ verb,
                                                   int32_t *__restrict__ target, int64_t *__restrict__ action,
                                                   float *__restrict__ logp) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t w0, w1;
    d1s::philox_w01(0u, t, (uint32_t)i, 3u, key0, key1, w0, w1);
    const float *vl = verb_logits + (size_t)i * ldv;
    float lv, lt;
    int v, tg;
    d1s::cat_core([&](int j) { return vl[j]; }, nv, d1s::unit24(w0), v, lv);
    const float *tl = target_logits + (size_t)i * ldt + (size_t)v * nt;
    d1s::cat_core([&](int j) { return tl[j]; }, nt, d1s::unit24(w1), tg, lt);
    if (verb) verb[i] = v;
    if (target) target[i] = tg;
    if (action) action[i] = d1s::ar_action(v, tg);
    if (logp) logp[i] = lv + lt;
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

// D4 camera transform of uint8 [n][15][15][8] observations: group g (0..7) mirrors x when
// g >= 4, then turns the window g % 4 quarter turns ((x, y) -> (-y, x) each, x east, y
// south, relative to the centre cell); out cell T_g(c) takes in cell c's 8 bytes. One
// lane per (env, cell) moves 8 bytes.
__global__ __launch_bounds__(256) void k_obs_d4(const uint8_t *__restrict__ obs, const int32_t *__restrict__ groups,
                                                int n, uint8_t *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)n * 225) return;
    const int env = (int)(i / 225), c = (int)(i - (int64_t)env * 225);
    const int g = groups[env] & 7;
    int x = c % 15 - 7, y = c / 15 - 7;
    if (g >= 4) x = -x;
    for (int r = 0; r < (g & 3); r++) {
        const int t = x;
        x = -y;
        y = t;
    }
    const uint64_t v = *(const uint64_t *)(obs + i * 8);
    *(uint64_t *)(out + ((int64_t)env * 225 + (y + 7) * 15 + x + 7) * 8) = v;
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
int d1_sample_dev(const float *logits, int n, int k, int ld, uint64_t seed, const uint32_t *t_dev, uint32_t t_add,
                  int64_t *actions, float *logp, void *stream) {
    if (n < 0 || k < 1 || k > 64 || ld < k || (n && (!logits || !t_dev))) return D1_E_ARG;
    if (n == 0) return 0;
    hipLaunchKernelGGL(d1p::k_sample_dev, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, logits, n, k, ld,
                       (uint32_t)seed, (uint32_t)(seed >> 32), t_dev, t_add, actions, logp);
    return (int)hipGetLastError();
}
int d1_obs_d4(const uint8_t *obs, const int32_t *groups, int n, uint8_t *out, void *stream) {
    if (n < 0 || (n && (!obs || !groups || !out)) || (uintptr_t)obs % 8 || (uintptr_t)out % 8) return D1_E_ARG;
    if (obs == out && n) return D1_E_ARG;   // a permutation needs a separate destination
    if (n == 0) return 0;
    const int64_t lanes = (int64_t)n * 225;
    hipLaunchKernelGGL(d1p::k_obs_d4, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, (hipStream_t)stream, obs,
                       groups, n, out);
    return (int)hipGetLastError();
}
int d1_sample_ar(const float *verb_logits, int nv, int ldv, const float *target_logits, int nt, int ldt, int n,
                 uint64_t seed, uint32_t t, int32_t *verb, int32_t *target, int64_t *action, float *logp,
                 void *stream) {
    if (n < 0 || nv < 1 || nv > 64 || nt < 1 || nt > 64 || ldv < nv || ldt < nv * nt) return D1_E_ARG;
    if (n && (!verb_logits || !target_logits)) return D1_E_ARG;
    if (n == 0) return 0;
    hipLaunchKernelGGL(d1p::k_sample_ar, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, verb_logits, nv,
                       ldv, target_logits, nt, ldt, n, (uint32_t)seed, (uint32_t)(seed >> 32), t, verb, target, action,
                       logp);
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
