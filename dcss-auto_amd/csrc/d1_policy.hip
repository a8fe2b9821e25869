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

// Two-stage (autoregressive) sample: verb ~ softmax(verb_logits[i]) with u0, then
// target ~ softmax(target_logits[i][verb]) with u1, where u0/u1 = words 0/1 of
// Philox4x32-10(ctr={0, t, i, 3}, key) scaled to [0,1) with 24 bits. logp = log p(verb) +
// log p(target | verb). Env action: verb 0 MOVE / 1 ATTACK with target (dx, dy) =
// (t%5-2, t/5-2) on a Chebyshev-1 ring -> direction d (N,E,S,W,NE,SE,SW,NW) -> d or 8+d,
// other targets -> -1 (one WAIT turn); verb 2 WAIT(16), 3 REST(17), 4 DESCEND(18), 5-7 WAIT.
__device__ __forceinline__ int cat_sample(const float *l, int k, float u, float &logp) {
    float m = l[0];
    for (int j = 1; j < k; j++) m = fmaxf(m, l[j]);
    float s = 0.f;
    for (int j = 0; j < k; j++) s += expf(l[j] - m);
    float c = 0.f;
    int a = k - 1;
    for (int j = 0; j < k; j++) {
        c += expf(l[j] - m) / s;
        if (u < c) { a = j; break; }
    }
    logp = l[a] - m - logf(s);
    return a;
}
__global__ __launch_bounds__(256) void k_sample_ar(const float *__restrict__ verb_logits, int nv, int ldv,
                                                   const float *__restrict__ target_logits, int nt, int ldt, int n,
                                                   uint32_t key0, uint32_t key1, uint32_t t, int32_t *__restrict__ verb,
                                                   int32_t *__restrict__ target, int64_t *__restrict__ action,
                                                   float *__restrict__ logp) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t c0 = 0u, c1 = t, c2 = (uint32_t)i, c3 = 3u, k0 = key0, k1 = key1;
#pragma unroll
    for (int r = 0; r < 10; r++) {
        uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
        uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
        uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
        k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
    }
    float u0 = (float)(c0 >> 8) * (1.0f / 16777216.0f), u1 = (float)(c1 >> 8) * (1.0f / 16777216.0f);
    float lv, lt;
    int v = cat_sample(verb_logits + (size_t)i * ldv, nv, u0, lv);
    int tg = cat_sample(target_logits + (size_t)i * ldt + (size_t)v * nt, nt, u1, lt);
    int a = 16;
    if (v <= 1) {
        int dx = tg % 5 - 2, dy = tg / 5 - 2, d = -1;
        if (dx == 0 && dy == -1) d = 0; else if (dx == 1 && dy == 0) d = 1; else if (dx == 0 && dy == 1) d = 2;
        else if (dx == -1 && dy == 0) d = 3; else if (dx == 1 && dy == -1) d = 4; else if (dx == 1 && dy == 1) d = 5;
        else if (dx == -1 && dy == 1) d = 6; else if (dx == -1 && dy == -1) d = 7;
        a = d < 0 ? -1 : d + 8 * v;
    } else if (v <= 4) a = 14 + v;
    if (verb) verb[i] = v;
    if (target) target[i] = tg;
    if (action) action[i] = a;
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

// ---------------------------------------------------------------- PPO minibatch kernels
// None of these clears memory with memset or reduces across workgroups through
// atomics, so a captured graph of a minibatch step replays exactly.
__device__ __forceinline__ float bf16_to_f(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }
__device__ __forceinline__ uint16_t f_to_bf16(float f) {   // round to nearest even
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u));
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Row gather of a minibatch: obs rows -> bf16 (exact), plus the per-sample scalars.
// One 128-lane workgroup per sample; `row_bytes` is a multiple of 8 (8 bytes in, 16 out per lane step).
__global__ __launch_bounds__(128) void k_ppo_gather(const uint8_t *__restrict__ obs, int row_bytes,
                                                    const int64_t *__restrict__ idx, const int64_t *__restrict__ act,
                                                    const float *__restrict__ logp, const float *__restrict__ adv,
                                                    const float *__restrict__ ret, uint16_t *__restrict__ xb,
                                                    int32_t *__restrict__ act_o, float *__restrict__ logp_o,
                                                    float *__restrict__ adv_o, float *__restrict__ ret_o) {
    int i = blockIdx.x;
    int64_t r = idx[i];
    const uint2 *src = (const uint2 *)(obs + (size_t)r * row_bytes);
    uint4 *dst = (uint4 *)(xb + (size_t)i * row_bytes);
    for (int c = threadIdx.x; c < row_bytes / 8; c += blockDim.x) {
        uint2 v = src[c];
        uint32_t w[2] = {v.x, v.y}, o[4];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            o[2 * j] = (__float_as_uint((float)(w[j] & 0xFFu)) >> 16) | (__float_as_uint((float)((w[j] >> 8) & 0xFFu)) & 0xFFFF0000u);
            o[2 * j + 1] = (__float_as_uint((float)((w[j] >> 16) & 0xFFu)) >> 16) | (__float_as_uint((float)(w[j] >> 24)) & 0xFFFF0000u);
        }
        dst[c] = make_uint4(o[0], o[1], o[2], o[3]);
    }
    if (threadIdx.x == 0) {
        act_o[i] = (int32_t)act[r];
        logp_o[i] = logp[r];
        adv_o[i] = adv[r];
        ret_o[i] = ret[r];
    }
}

// Clipped-surrogate + value + entropy loss and its gradient w.r.t. the head output
// z = [logits(k) | value] (bf16, row stride ldz). Per sample, with p = softmax(logits),
// r = exp(logp_a - old):
//   dL/dz_j = (g_r * r * ([j==a] - p_j) + ecoef * p_j * (log p_j + H)) / mb,
//   g_r = -A when r*A <= clip(r)*A (torch.minimum routes ties to its first argument), else 0;
//   dL/dvalue = vcoef * (v - R) / mb.
// partial[b*4 + {0,1,2}] = this workgroup's sums of the per-sample pg, 0.5*(v-R)^2, H.
__global__ __launch_bounds__(256) void k_ppo_loss(const uint16_t *__restrict__ z, int ldz, int k,
                                                  const int32_t *__restrict__ act, const float *__restrict__ old_logp,
                                                  const float *__restrict__ adv, const float *__restrict__ ret, int mb,
                                                  float clip, float vcoef, float ecoef, uint16_t *__restrict__ dz,
                                                  float *__restrict__ partial) {
    __shared__ float red[3][256];
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    float pg = 0.f, vl = 0.f, ent = 0.f;
    if (i < mb) {
        constexpr int KMAX = 32;
        const uint16_t *zi = z + (size_t)i * ldz;
        float l[KMAX];
        float m = -3.0e38f;
#pragma unroll
        for (int j = 0; j < KMAX; j++) { l[j] = j < k ? bf16_to_f(zi[j]) : -3.0e38f; m = fmaxf(m, l[j]); }
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < KMAX; j++) s += j < k ? expf(l[j] - m) : 0.f;
        float ls = logf(s);
        int a = act[i];
        float h = 0.f, la = 0.f;
#pragma unroll
        for (int j = 0; j < KMAX; j++) {
            if (j < k) { float lp = l[j] - m - ls; h -= expf(lp) * lp; }
            if (j == a) la = l[j];
        }
        float lpa = la - m - ls;
        float r = expf(lpa - old_logp[i]);
        float A = adv[i];
        float un = r * A, cl = fminf(fmaxf(r, 1.f - clip), 1.f + clip) * A;
        pg = -fminf(un, cl);
        float gr = un <= cl ? -A : 0.f;
        float v = bf16_to_f(zi[k]), d = v - ret[i];
        vl = 0.5f * d * d;
        ent = h;
        float inv = 1.f / (float)mb;
        uint16_t *di = dz + (size_t)i * ldz;
#pragma unroll
        for (int j = 0; j < KMAX; j++) {
            if (j < k) {
                float lp = l[j] - m - ls, p = expf(lp);
                float g = gr * r * ((j == a ? 1.f : 0.f) - p) + ecoef * p * (lp + h);
                di[j] = f_to_bf16(g * inv);
            }
        }
        di[k] = f_to_bf16(vcoef * d * inv);
    }
    red[0][threadIdx.x] = pg; red[1][threadIdx.x] = vl; red[2][threadIdx.x] = ent;
    __syncthreads();
    for (int o = blockDim.x / 2; o; o >>= 1) {
        if ((int)threadIdx.x < o)
            for (int q = 0; q < 3; q++) red[q][threadIdx.x] += red[q][threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x < 3) partial[blockIdx.x * 4 + threadIdx.x] = red[threadIdx.x][0];
}

// dh *= (h > 0), bf16, in place (ReLU backward).
__global__ __launch_bounds__(256) void k_relu_bwd(uint16_t *__restrict__ dh, const uint16_t *__restrict__ h, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n && !(bf16_to_f(h[i]) > 0.f)) dh[i] = 0;
}

// ReLU backward fused with the bias gradient: dh *= (h > 0) on a [rows, cols] bf16 block
// (cols <= 256), and colpart[b*cols + c] = sum over this workgroup's rows of the masked dh.
// Workgroup = 256 lanes, lane = column; rows split in chunks of `rows_per`.
__global__ __launch_bounds__(256) void k_relu_bwd_bias(uint16_t *__restrict__ dh, const uint16_t *__restrict__ h,
                                                       int rows, int cols, int rows_per, float *__restrict__ colpart) {
    int c = threadIdx.x;
    int r0 = blockIdx.x * rows_per, r1 = min(rows, r0 + rows_per);
    float acc = 0.f;
    if (c < cols) {
        for (int r = r0; r < r1; r++) {
            size_t o = (size_t)r * cols + c;
            float v = bf16_to_f(dh[o]);
            if (!(bf16_to_f(h[o]) > 0.f)) { v = 0.f; dh[o] = 0; }
            acc += v;
        }
        colpart[(size_t)blockIdx.x * cols + c] = acc;
    }
}
// Column sums of a [rows, cols] bf16 block into colpart (no masking).
__global__ __launch_bounds__(256) void k_colsum(const uint16_t *__restrict__ x, int rows, int cols, int ld,
                                                int rows_per, float *__restrict__ colpart) {
    int c = threadIdx.x;
    int r0 = blockIdx.x * rows_per, r1 = min(rows, r0 + rows_per);
    if (c < cols) {
        float acc = 0.f;
        for (int r = r0; r < r1; r++) acc += bf16_to_f(x[(size_t)r * ld + c]);
        colpart[(size_t)blockIdx.x * cols + c] = acc;
    }
}
// out[c] = bf16(sum_b colpart[b*cols + c]); one workgroup per column, tree sum in LDS.
__global__ __launch_bounds__(256) void k_colsum_finish(const float *__restrict__ colpart, int nblocks, int cols,
                                                       uint16_t *__restrict__ out) {
    __shared__ float red[256];
    int c = blockIdx.x;
    float acc = 0.f;
    for (int b = threadIdx.x; b < nblocks; b += blockDim.x) acc += colpart[(size_t)b * cols + c];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int o = blockDim.x / 2; o; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[c] = f_to_bf16(red[0]);
}
// out[j] = bf16(sum_s part[s*n + j]) over S split-K partials (bf16), 8 elements per lane.
__global__ __launch_bounds__(256) void k_sum_partials(const uint16_t *__restrict__ part, int S, size_t n,
                                                      uint16_t *__restrict__ out) {
    size_t j = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (j >= n) return;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (j + 8 <= n && (n % 8) == 0) {
        for (int q = 0; q < S; q++) {
            uint4 v = *(const uint4 *)(part + (size_t)q * n + j);
            uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; e++) { acc[2 * e] += bf16_to_f((uint16_t)w[e]); acc[2 * e + 1] += bf16_to_f((uint16_t)(w[e] >> 16)); }
        }
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; e++) o[e] = (uint32_t)f_to_bf16(acc[2 * e]) | ((uint32_t)f_to_bf16(acc[2 * e + 1]) << 16);
        *(uint4 *)(out + j) = make_uint4(o[0], o[1], o[2], o[3]);
    } else {
        for (size_t k = j; k < n && k < j + 8; k++) {
            float a = 0.f;
            for (int q = 0; q < S; q++) a += bf16_to_f(part[(size_t)q * n + k]);
            out[k] = f_to_bf16(a);
        }
    }
}

// Sum of squares of the bf16 gradient buffer: one partial per workgroup.
__global__ __launch_bounds__(256) void k_sqnorm(const uint16_t *__restrict__ g, size_t n, float *__restrict__ partial,
                                                float *__restrict__ step) {
    if (blockIdx.x == 0 && threadIdx.x == 0) step[1] = step[0] + 1.f;   // t for the Adam launch that follows
    __shared__ float red[256];
    float acc = 0.f;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        float v = bf16_to_f(g[i]);
        acc += v * v;
    }
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int o = blockDim.x / 2; o; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

// Gradient-norm clipping + Adam (torch.optim.Adam, no weight decay) over flat buffers.
// Every workgroup re-sums the `nparts` norm partials (so no cross-workgroup handoff),
// takes coef = min(max_norm / (||g|| + 1e-6), 1), and updates its slice. The step count:
// k_sqnorm wrote t = step[0] + 1 to step[1]; every workgroup here reads step[1] and
// workgroup 0 stores it back to step[0] for the next call.
__global__ __launch_bounds__(256) void k_adam(float *__restrict__ p, uint16_t *__restrict__ pb,
                                              const uint16_t *__restrict__ g, float *__restrict__ m,
                                              float *__restrict__ v, size_t n, const float *__restrict__ partial,
                                              int nparts, float max_norm, float lr, float b1, float b2, float eps,
                                              float *__restrict__ step) {
    __shared__ float red[256];
    float acc = 0.f;
    for (int j = threadIdx.x; j < nparts; j += blockDim.x) acc += partial[j];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int o = blockDim.x / 2; o; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    float norm = sqrtf(red[0]);
    float coef = fminf(max_norm / (norm + 1e-6f), 1.f);
    float t = step[1];
    float bc1 = 1.f - powf(b1, t), bc2 = 1.f - powf(b2, t);
    float step_size = lr / bc1, bc2s = sqrtf(bc2);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        float gi = bf16_to_f(g[i]) * coef;
        float mi = b1 * m[i] + (1.f - b1) * gi;
        float vi = b2 * v[i] + (1.f - b2) * gi * gi;
        m[i] = mi;
        v[i] = vi;
        float pi = p[i] - step_size * mi / (sqrtf(vi) / bc2s + eps);
        p[i] = pi;
        pb[i] = f_to_bf16(pi);
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) step[0] = t;
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
int d1_ppo_gather(const uint8_t *obs, int row_bytes, const int64_t *idx, int mb, const int64_t *act,
                  const float *logp, const float *adv, const float *ret, void *xb, int32_t *act_o, float *logp_o,
                  float *adv_o, float *ret_o, void *stream) {
    if (mb < 0 || row_bytes <= 0 || (row_bytes % 8)) return D1_E_ARG;
    if (mb && (!obs || !idx || !act || !logp || !adv || !ret || !xb || !act_o || !logp_o || !adv_o || !ret_o))
        return D1_E_ARG;
    if (mb == 0) return 0;
    hipLaunchKernelGGL(d1p::k_ppo_gather, dim3(mb), dim3(128), 0, (hipStream_t)stream, obs, row_bytes, idx, act, logp,
                       adv, ret, (uint16_t *)xb, act_o, logp_o, adv_o, ret_o);
    return (int)hipGetLastError();
}
int d1_ppo_loss(const void *z, int ldz, int k, const int32_t *act, const float *old_logp, const float *adv,
                const float *ret, int mb, float clip, float vcoef, float ecoef, void *dz, float *partial,
                void *stream) {
    if (mb < 0 || k < 1 || k > 32 || ldz < k + 1) return D1_E_ARG;
    if (mb && (!z || !act || !old_logp || !adv || !ret || !dz || !partial)) return D1_E_ARG;
    if (mb == 0) return 0;
    hipLaunchKernelGGL(d1p::k_ppo_loss, dim3((mb + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t *)z, ldz, k, act, old_logp, adv, ret, mb, clip, vcoef, ecoef, (uint16_t *)dz,
                       partial);
    return (int)hipGetLastError();
}
int d1_relu_bwd(void *dh, const void *h, int64_t n, void *stream) {
    if (n < 0 || (n && (!dh || !h))) return D1_E_ARG;
    if (n == 0) return 0;
    hipLaunchKernelGGL(d1p::k_relu_bwd, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (uint16_t *)dh, (const uint16_t *)h, (size_t)n);
    return (int)hipGetLastError();
}
int d1_relu_bwd_bias(void *dh, const void *h, int rows, int cols, float *colpart, int nblocks, void *bias_grad,
                     void *stream) {
    if (rows <= 0 || cols <= 0 || cols > 256 || nblocks < 1 || !dh || !h || !colpart || !bias_grad) return D1_E_ARG;
    int per = (rows + nblocks - 1) / nblocks;
    hipLaunchKernelGGL(d1p::k_relu_bwd_bias, dim3(nblocks), dim3(256), 0, (hipStream_t)stream, (uint16_t *)dh,
                       (const uint16_t *)h, rows, cols, per, colpart);
    hipLaunchKernelGGL(d1p::k_colsum_finish, dim3(cols), dim3(256), 0, (hipStream_t)stream, colpart, nblocks, cols,
                       (uint16_t *)bias_grad);
    return (int)hipGetLastError();
}
int d1_colsum(const void *x, int rows, int cols, int ld, float *colpart, int nblocks, void *out, void *stream) {
    if (rows <= 0 || cols <= 0 || cols > 256 || ld < cols || nblocks < 1 || !x || !colpart || !out) return D1_E_ARG;
    int per = (rows + nblocks - 1) / nblocks;
    hipLaunchKernelGGL(d1p::k_colsum, dim3(nblocks), dim3(256), 0, (hipStream_t)stream, (const uint16_t *)x, rows,
                       cols, ld, per, colpart);
    hipLaunchKernelGGL(d1p::k_colsum_finish, dim3(cols), dim3(256), 0, (hipStream_t)stream, colpart, nblocks, cols,
                       (uint16_t *)out);
    return (int)hipGetLastError();
}
int d1_sum_partials(const void *part, int S, int64_t n, void *out, void *stream) {
    if (S < 1 || n <= 0 || !part || !out) return D1_E_ARG;
    size_t threads = ((size_t)n + 7) / 8;
    hipLaunchKernelGGL(d1p::k_sum_partials, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t *)part, S, (size_t)n, (uint16_t *)out);
    return (int)hipGetLastError();
}
int d1_adam_clip(float *p, void *pb, const void *g, float *m, float *v, int64_t n, float *partial, int nparts,
                 float max_norm, float lr, float b1, float b2, float eps, float *step, void *stream) {
    if (n <= 0 || nparts < 1 || nparts > 4096 || !p || !pb || !g || !m || !v || !partial || !step)
        return D1_E_ARG;
    hipLaunchKernelGGL(d1p::k_sqnorm, dim3(nparts), dim3(256), 0, (hipStream_t)stream, (const uint16_t *)g, (size_t)n,
                       partial, step);
    hipLaunchKernelGGL(d1p::k_adam, dim3(nparts), dim3(256), 0, (hipStream_t)stream, p, (uint16_t *)pb,
                       (const uint16_t *)g, m, v, (size_t)n, partial, nparts, max_norm, lr, b1, b2, eps, step);
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
