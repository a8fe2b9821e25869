// d1hip: the PPO minibatch update as four kernels for MI355X (gfx950).
//
// One d1_ppo_step call is one minibatch of the clipped-surrogate update
// (gpu-d1/scripts/train_clear.py:160-172, gpu-d1/scripts/run_ring_ablations.py:363-372) for
// the 1800 -> 256 -> 256 ReLU policy with a 17-wide head (16 logits + value), computed as
// torch bf16 autocast does it: bf16 operands, fp32 accumulation, bf16 results, fp32 masters.
//
//   k_rows    one 512-lane workgroup per 32 samples. Gathers through the sample order, then
//             h1 = relu(x W1^T + b1) straight from the uint8 rows, h2 = relu(h1 W2^T + b2),
//             z = h2 W3^T + b3, the loss and dL/dz, dh2 = (dz W3)[h2 > 0] and
//             dh1 = (dh2 W2)[h1 > 0], with per-workgroup bias-gradient and loss partials.
//             Wave w owns columns 32w..32w+31 of every layer; activations cross waves through
//             LDS, and leave for the weight gradients as [feature][sample] bf16 arrays.
//   k_wgrad   dW1 = dh1^T x, dW2 = dh2^T h1, dW3 = dz^T h2 in one grouped launch of split-K
//             MFMA tiles with fp32 partials. x is re-read through the sample order and
//             transposed to [feature][sample] through LDS.
//   k_reduce  fixed-order sums of the partials -> bf16 gradients (one rounding, as the bf16
//             GEMM gives), and sum-of-squares partials for the clipping norm.
//   k_adam    global-norm clip + Adam on the fp32 masters, the bf16 copy, the transposed
//             W2 / W3 copies the next k_rows reads, and the minibatch cursor.
//
// MFMA: v_mfma_f32_32x32x16_bf16. Lane layouts (checked on the hardware): A lane l holds
// A[l%32][8(l/32)+j], B lane l holds B[8(l/32)+j][l%32], D lane l holds
// D[8(r/4)+4(l/32)+r%4][l%32]. The contraction order inside a 64-wide K chunk is free as
// long as A and B agree, so in chunk k0, step q, slot j of a lane in half h stands for
// k = k0 + 32h + 8q + j: each lane then reads 32 contiguous K values per operand row.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/d1hip.h"

namespace d1q {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16;

constexpr int K1 = 1800;              // observation bytes = layer-1 inputs
constexpr int H = 256;                // hidden width
constexpr int NA = 16, NZ = 17;       // logits, head width
constexpr int R = 32;                 // samples per k_rows workgroup
constexpr int XS = H + 8;             // LDS row stride (bf16) of the [32][256] activation tiles
constexpr int DS = 40;                // LDS row stride (bf16) of the dz tile (32 columns used)
constexpr int BP = 544;               // bias partial row: db1[256] | db2[256] | db3[17] | pad
constexpr int KW = 1024;              // samples per dW1 / dW2 workgroup
constexpr int KW3 = 512;              // samples per dW3 workgroup
constexpr int NT1 = (K1 + 63) / 64;   // dW1 column tiles of 64 (the last one holds 8 columns)
constexpr int XR = K1 + 8;            // LDS row stride (bytes) of k_rows' x tile
constexpr int NRED = 512;             // k_reduce weight workgroups (+ NBIAS for the biases)
constexpr int NBIASB = (2 * H + NZ + 63) / 64;   // k_reduce bias workgroups (64 columns each)
constexpr int NADAM = 1024;           // k_adam workgroups

struct Work {
    uint16_t *h1t, *h2t, *dh2t, *dh1t;   // [256][mb] bf16
    uint16_t *dzt;                       // [17][mb] bf16
    uint8_t *xt;                         // [1800][mb] the minibatch's observations, transposed
    float *bpart;                        // [mb/32][BP]
    float *part1, *part2, *part3;        // [S1][256][1800], [S1][256][256], [S3][17][256]
    float *npart;                        // [NRED + NBIASB] sum-of-squares partials
};

__device__ __forceinline__ float bf(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }
__device__ __forceinline__ uint16_t rb(float f) {   // float -> bf16, round to nearest even
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u));
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
// two bytes of x (at bit 8s) -> two bf16 in one dword (exact: byte values need 8 bits)
__device__ __forceinline__ uint32_t widen2(uint32_t x, int s) {
    uint32_t lo = __float_as_uint((float)((x >> (8 * s)) & 255u)) >> 16;
    uint32_t hi = __float_as_uint((float)((x >> (8 * s + 8)) & 255u)) & 0xFFFF0000u;
    return lo | hi;
}
__device__ __forceinline__ bf16x8 widen8(uint32_t x0, uint32_t x1) {
    return __builtin_bit_cast(bf16x8, make_uint4(widen2(x0, 0), widen2(x0, 2), widen2(x1, 0), widen2(x1, 2)));
}
__device__ __forceinline__ bf16x8 as_bf(uint4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ floatx16 mfma(bf16x8 a, bf16x8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ int64_t clamp_index(int64_t s, int64_t n) { return s < 0 ? 0 : (s >= n ? n - 1 : s); }
__device__ __forceinline__ bool cursor_ok(const D1PPOStep &a) {
    const int cur = a.cursor[0];
    return cur >= 0 && (int64_t)(cur + 1) * a.mb <= a.n;
}
// D row of accumulator register r in lane half h
__device__ __forceinline__ int drow(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// ---------------------------------------------------------------- k_rows
// Epilogue shared by the four row-block products: v[r] (fp32, this lane's column c) ->
// bf16 bits, LDS row-major tile (if any), the [c][sample] global array, bit r of *mask set
// where the bf16 value is > 0 (if asked), and the column sum of the bf16 values (lanes < 32
// hold the full 32-row sum afterwards).
__device__ __forceinline__ float rows_out(const float (&v)[16], uint16_t *tile, uint16_t *gt, int mb, int m0, int c,
                                          int lh, uint32_t *mask) {
    uint16_t hb[16];
    float colsum = 0.f;
    uint32_t pos = 0;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        hb[r] = rb(v[r]);
        colsum += bf(hb[r]);
        if (bf(hb[r]) > 0.f) pos |= 1u << r;
        if (tile) tile[drow(r, lh) * XS + c] = hb[r];
    }
    if (mask) *mask = pos;
#pragma unroll
    for (int g = 0; g < 4; g++)   // rows 8g + 4h .. +3 are registers 4g .. 4g+3
        *(uint2 *)(gt + (size_t)c * mb + m0 + 8 * g + 4 * lh) =
            make_uint2((uint32_t)hb[4 * g] | ((uint32_t)hb[4 * g + 1] << 16),
                       (uint32_t)hb[4 * g + 2] | ((uint32_t)hb[4 * g + 3] << 16));
    return colsum + __shfl_xor(colsum, 32);
}

__global__ __launch_bounds__(512) void k_rows(D1PPOStep a, Work w) {
    // The 32 x rows (layer 1) share their LDS with the tiles of the later phases.
    __shared__ __align__(16) uint8_t lds[R * XR];
    uint8_t *xs = lds;                                                       // x rows, stride XR
    uint16_t *x1 = (uint16_t *)lds;                                          // h1, later dh2 (row-major)
    uint16_t *x2 = (uint16_t *)(lds + R * XS * 2);                           // h2
    uint16_t *dzs = (uint16_t *)(lds + 2 * R * XS * 2);                      // dL/dz, columns 17..31 zero
    float(*zp)[R][NZ] = (float(*)[R][NZ])(lds + 2 * R * XS * 2 + R * DS * 2);   // head partials per wave
    static_assert(2 * R * XS * 2 + R * DS * 2 + 8 * R * NZ * 4 <= R * XR, "LDS union");
    __shared__ int64_t srow[R];
    __shared__ float sold[R], sadv[R], sret[R];
    __shared__ int sact[R];
    if (!cursor_ok(a)) return;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, lr = lane & 31, lh = lane >> 5;
    const int mb = a.mb, m0 = blockIdx.x * R;
    const int64_t base = (int64_t)a.cursor[0] * mb + m0;
    const uint16_t *pb = (const uint16_t *)a.pb;
    const uint16_t *W1 = pb + a.off_w1, *B1 = pb + a.off_b1, *W2 = pb + a.off_w2, *B2 = pb + a.off_b2;
    const uint16_t *W3 = pb + a.off_w3, *B3 = pb + a.off_b3;
    const uint16_t *W2T = (const uint16_t *)a.w2t, *W3T = (const uint16_t *)a.w3t;
    if (t < R) {
        const int64_t s = clamp_index(a.perm[base + t], a.n);   // entries outside [0, n) are a caller error
        srow[t] = s;
        sact[t] = (int)a.actions[s];
        sold[t] = a.logp_old[s];
        sadv[t] = a.adv[s];
        sret[t] = a.ret[s];
    }
    __syncthreads();
    {   // the 32 observation rows -> LDS: every load in flight at once
        constexpr int XU = K1 / 8, NU = (R * XU + 511) / 512;
        uint2 tmp[NU];
#pragma unroll
        for (int i = 0; i < NU; i++) {
            const int u = t + 512 * i, r = u / XU, cc = u - r * XU;
            tmp[i] = u < R * XU ? *(const uint2 *)(a.obs + srow[r] * K1 + 8 * cc) : make_uint2(0u, 0u);
        }
#pragma unroll
        for (int i = 0; i < NU; i++) {
            const int u = t + 512 * i, r = u / XU, cc = u - r * XU;
            if (u < R * XU) *(uint2 *)(xs + r * XR + 8 * cc) = tmp[i];
        }
    }
    __syncthreads();
    // x^T for the dW1 product: xt[k][m0 + r], 4 inputs x 4 samples per unit, transposed in registers
    for (int u = t; u < (K1 / 4) * (R / 4); u += 512) {
        const int rg = u & 7, kg = u >> 3;
        uint32_t x[4];
#pragma unroll
        for (int i = 0; i < 4; i++) x[i] = *(const uint32_t *)(xs + (4 * rg + i) * XR + 4 * kg);
#pragma unroll
        for (int e = 0; e < 4; e++)
            *(uint32_t *)(w.xt + (size_t)(4 * kg + e) * mb + m0 + 4 * rg) =
                ((x[0] >> (8 * e)) & 255u) | (((x[1] >> (8 * e)) & 255u) << 8) | (((x[2] >> (8 * e)) & 255u) << 16) |
                (((x[3] >> (8 * e)) & 255u) << 24);
    }
    const int c = 32 * wave + lr;   // this lane's column in every layer
    float v[16];

    // ---- layer 1: 28 chunks of 64 inputs (A from the LDS rows, W1 through a 4-deep register
    // ring, loads issued 3 chunks ahead), then k = 1792..1799 (lower half, q = 0)
    uint32_t mask1 = 0, mask2 = 0;
    {
        const uint8_t *xr = xs + lr * XR + 32 * lh;
        const uint16_t *wr = W1 + (size_t)c * K1 + 32 * lh;
        floatx16 e0 = {}, e1 = {};
        uint4 wb[4][4];
        auto wload = [&](uint4 (&dst)[4], int ch) {
#pragma unroll
            for (int q = 0; q < 4; q++) dst[q] = *(const uint4 *)(wr + 64 * ch + 8 * q);
        };
        wload(wb[0], 0);
        wload(wb[1], 1);
        wload(wb[2], 2);
        for (int ch0 = 0; ch0 < 28; ch0 += 4) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int ch = ch0 + u;
                if (ch + 3 < 28) wload(wb[(u + 3) & 3], ch + 3);
                const uint4 lo = *(const uint4 *)(xr + 64 * ch), hi = *(const uint4 *)(xr + 64 * ch + 16);
                e0 = mfma(widen8(lo.x, lo.y), as_bf(wb[u][0]), e0);
                e1 = mfma(widen8(lo.z, lo.w), as_bf(wb[u][1]), e1);
                e0 = mfma(widen8(hi.x, hi.y), as_bf(wb[u][2]), e0);
                e1 = mfma(widen8(hi.z, hi.w), as_bf(wb[u][3]), e1);
            }
        }
        const uint2 xt = lh == 0 ? *(const uint2 *)(xs + lr * XR + 1792) : make_uint2(0u, 0u);
        const uint4 wt = lh == 0 ? *(const uint4 *)(W1 + (size_t)c * K1 + 1792) : make_uint4(0u, 0u, 0u, 0u);
        e0 = mfma(widen8(xt.x, xt.y), as_bf(wt), e0);
        __syncthreads();   // every wave is done with the x rows before h1 overwrites them
        const float bias = bf(B1[c]);
#pragma unroll
        for (int r = 0; r < 16; r++) v[r] = fmaxf(e0[r] + e1[r] + bias, 0.f);
        rows_out(v, x1, w.h1t, mb, m0, c, lh, &mask1);
    }
    __syncthreads();

    // ---- layer 2: h2 = relu(h1 W2^T + b2), K = 256 from the LDS h1 tile
    {
        const uint16_t *ar = x1 + lr * XS + 32 * lh;
        const uint16_t *br = W2 + (size_t)c * H + 32 * lh;
        floatx16 e0 = {}, e1 = {};
#pragma unroll
        for (int k0 = 0; k0 < H; k0 += 64) {
            bf16x8 fa[4], fb[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                fa[q] = as_bf(*(const uint4 *)(ar + k0 + 8 * q));
                fb[q] = as_bf(*(const uint4 *)(br + k0 + 8 * q));
            }
            e0 = mfma(fa[0], fb[0], e0);
            e1 = mfma(fa[1], fb[1], e1);
            e0 = mfma(fa[2], fb[2], e0);
            e1 = mfma(fa[3], fb[3], e1);
        }
        const float bias = bf(B2[c]);
#pragma unroll
        for (int r = 0; r < 16; r++) v[r] = fmaxf(e0[r] + e1[r] + bias, 0.f);
        rows_out(v, x2, w.h2t, mb, m0, c, lh, &mask2);
    }
    __syncthreads();

    // ---- head partials: wave w contracts k = 32w..32w+31 (two K16 steps, slot 8h+j <-> k = 32w+16s+8h+j)
    {
        floatx16 zacc = {};
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int k = 32 * wave + 16 * s + 8 * lh;
            const uint4 av = *(const uint4 *)(x2 + lr * XS + k);
            const uint4 bv = lr < NZ ? *(const uint4 *)(W3 + (size_t)lr * H + k) : make_uint4(0u, 0u, 0u, 0u);
            zacc = mfma(as_bf(av), as_bf(bv), zacc);
        }
        if (lr < NZ) {
#pragma unroll
            for (int r = 0; r < 16; r++) zp[wave][drow(r, lh)][lr] = zacc[r];
        }
    }
    __syncthreads();

    // ---- loss and dL/dz: wave 0, lane = sample (k_ppo formula, k = 16 logits)
    if (wave == 0) {
        float pg = 0.f, vl = 0.f, ent = 0.f;
        if (lane < R) {
            const int r = lane;
            float l[NZ];
#pragma unroll
            for (int j = 0; j < NZ; j++) {
                float s = zp[0][r][j];
#pragma unroll
                for (int q = 1; q < 8; q++) s += zp[q][r][j];
                l[j] = bf(rb(s + bf(B3[j])));   // the head output is bf16
            }
            float mx = l[0];
#pragma unroll
            for (int j = 1; j < NA; j++) mx = fmaxf(mx, l[j]);
            float se = 0.f;
#pragma unroll
            for (int j = 0; j < NA; j++) se += expf(l[j] - mx);
            const float ls = logf(se);
            const int act = sact[r];
            float hh = 0.f, la = 0.f;
#pragma unroll
            for (int j = 0; j < NA; j++) {
                const float lp = l[j] - mx - ls;
                hh -= expf(lp) * lp;
                if (j == act) la = l[j];
            }
            const float lpa = la - mx - ls;
            const float ratio = expf(lpa - sold[r]);
            const float A = sadv[r];
            const float un = ratio * A, cl = fminf(fmaxf(ratio, 1.f - a.clip), 1.f + a.clip) * A;
            pg = -fminf(un, cl);
            const float gr = un <= cl ? -A : 0.f;   // torch.minimum routes ties to its first argument
            const float d = l[NA] - sret[r];
            vl = 0.5f * d * d;
            ent = hh;
            const float inv = 1.f / (float)mb;
            uint16_t dz[32];
#pragma unroll
            for (int j = 0; j < NA; j++) {
                const float lp = l[j] - mx - ls, p = expf(lp);
                const float gj = gr * ratio * ((j == act ? 1.f : 0.f) - p) + a.ecoef * p * (lp + hh);
                dz[j] = rb(gj * inv);
            }
            dz[NA] = rb(a.vcoef * d * inv);
#pragma unroll
            for (int j = NZ; j < 32; j++) dz[j] = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                uint4 u;
                u.x = (uint32_t)dz[8 * q] | ((uint32_t)dz[8 * q + 1] << 16);
                u.y = (uint32_t)dz[8 * q + 2] | ((uint32_t)dz[8 * q + 3] << 16);
                u.z = (uint32_t)dz[8 * q + 4] | ((uint32_t)dz[8 * q + 5] << 16);
                u.w = (uint32_t)dz[8 * q + 6] | ((uint32_t)dz[8 * q + 7] << 16);
                *(uint4 *)(dzs + r * DS + 8 * q) = u;
            }
#pragma unroll
            for (int j = 0; j < NZ; j++) w.dzt[(size_t)j * mb + m0 + r] = dz[j];
        }
#pragma unroll
        for (int o = 32; o; o >>= 1) {
            pg += __shfl_xor(pg, o);
            vl += __shfl_xor(vl, o);
            ent += __shfl_xor(ent, o);
        }
        if (lane == 0) {
            float *lp = a.loss_parts + (size_t)blockIdx.x * 4;
            lp[0] = pg;
            lp[1] = vl;
            lp[2] = ent;
            lp[3] = 0.f;
        }
    }
    __syncthreads();
    if (t < NZ) {   // head-bias partial
        float s = 0.f;
        for (int r = 0; r < R; r++) s += bf(dzs[r * DS + t]);
        w.bpart[(size_t)blockIdx.x * BP + 2 * H + t] = s;
    }

    // ---- dh2 = (dz W3)[h2 > 0]: K = 17 padded to 32, B = W3^T rows
    {
        floatx16 acc = {};
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const uint4 av = *(const uint4 *)(dzs + lr * DS + 16 * s + 8 * lh);
            const uint4 bv = *(const uint4 *)(W3T + (size_t)c * 32 + 16 * s + 8 * lh);
            acc = mfma(as_bf(av), as_bf(bv), acc);
        }
#pragma unroll
        for (int r = 0; r < 16; r++) v[r] = (mask2 >> r) & 1u ? acc[r] : 0.f;
        const float cs = rows_out(v, x1, w.dh2t, mb, m0, c, lh, nullptr);
        if (lh == 0) w.bpart[(size_t)blockIdx.x * BP + H + c] = cs;
    }
    __syncthreads();

    // ---- dh1 = (dh2 W2)[h1 > 0]: K = 256 from the LDS dh2 tile, B = W2^T rows
    {
        const uint16_t *ar = x1 + lr * XS + 32 * lh;
        const uint16_t *br = W2T + (size_t)c * H + 32 * lh;
        floatx16 e0 = {}, e1 = {};
#pragma unroll
        for (int k0 = 0; k0 < H; k0 += 64) {
            bf16x8 fa[4], fb[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                fa[q] = as_bf(*(const uint4 *)(ar + k0 + 8 * q));
                fb[q] = as_bf(*(const uint4 *)(br + k0 + 8 * q));
            }
            e0 = mfma(fa[0], fb[0], e0);
            e1 = mfma(fa[1], fb[1], e1);
            e0 = mfma(fa[2], fb[2], e0);
            e1 = mfma(fa[3], fb[3], e1);
        }
#pragma unroll
        for (int r = 0; r < 16; r++) v[r] = (mask1 >> r) & 1u ? e0[r] + e1[r] : 0.f;
        const float cs = rows_out(v, nullptr, w.dh1t, mb, m0, c, lh, nullptr);
        if (lh == 0) w.bpart[(size_t)blockIdx.x * BP + c] = cs;
    }
}

// ---------------------------------------------------------------- k_wgrad
// One split-K tile of out[i][j] = sum_m at[i][m] bt[j][m] over samples [ms, ms + ks): both
// operands are [row][sample] (K-contiguous); `at` bf16, `bt` bf16 or (XB) uint8. Wave w owns
// NA_ row blocks of 32 from i0, the workgroup's NB_ column blocks of 32 from j0; rows past
// arows / brows read as zero. Loads run through a RING-deep register ring (issued RING-1
// chunks of 64 samples ahead); ks / 64 is a multiple of RING.
template <int NA_, int NB_, bool XB, int RING>
__device__ __forceinline__ void wgrad_tile(const uint16_t *at, int arows, int i0, const void *bt, int brows, int j0,
                                           int mb, int ms, int ks, floatx16 (&acc)[NA_][NB_]) {
    constexpr int BW = XB ? 2 : 4;   // uint4 per B row and chunk
    const int lane = threadIdx.x & 63, lr = lane & 31, lh = lane >> 5;
    const uint16_t *ar[NA_];
    bool aok[NA_];
#pragma unroll
    for (int i = 0; i < NA_; i++) {
        aok[i] = i0 + 32 * i + lr < arows;
        ar[i] = at + (size_t)(aok[i] ? i0 + 32 * i + lr : 0) * mb + ms + 32 * lh;
    }
    const uint4 *br[NB_];
    bool bok[NB_];
#pragma unroll
    for (int b = 0; b < NB_; b++) {
        bok[b] = j0 + 32 * b + lr < brows;
        const size_t row = bok[b] ? j0 + 32 * b + lr : 0;
        br[b] = XB ? (const uint4 *)((const uint8_t *)bt + row * mb + ms + 32 * lh)
                   : (const uint4 *)((const uint16_t *)bt + row * mb + ms + 32 * lh);
    }
    uint4 av[RING][NA_][4], bv[RING][NB_][BW];
    auto load = [&](int slot, int ch) {
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int i = 0; i < NA_; i++)
                av[slot][i][q] = aok[i] ? *(const uint4 *)(ar[i] + 64 * ch + 8 * q) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int q = 0; q < BW; q++)
#pragma unroll
            for (int b = 0; b < NB_; b++)
                bv[slot][b][q] = bok[b] ? br[b][(XB ? 4 : 8) * ch + q] : make_uint4(0u, 0u, 0u, 0u);
    };
    const int nch = ks / 64;
#pragma unroll
    for (int u = 0; u + 1 < RING; u++) load(u, u);
    for (int ch0 = 0; ch0 < nch; ch0 += RING) {
#pragma unroll
        for (int u = 0; u < RING; u++) {
            const int ch = ch0 + u;
            if (ch + RING - 1 < nch) load((u + RING - 1) % RING, ch + RING - 1);
            bf16x8 fb[NB_][4];
#pragma unroll
            for (int b = 0; b < NB_; b++) {
                if (XB) {
                    fb[b][0] = widen8(bv[u][b][0].x, bv[u][b][0].y);
                    fb[b][1] = widen8(bv[u][b][0].z, bv[u][b][0].w);
                    fb[b][2] = widen8(bv[u][b][1].x, bv[u][b][1].y);
                    fb[b][3] = widen8(bv[u][b][1].z, bv[u][b][1].w);
                } else {
#pragma unroll
                    for (int q = 0; q < 4; q++) fb[b][q] = as_bf(bv[u][b][q]);
                }
            }
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int i = 0; i < NA_; i++)
#pragma unroll
                    for (int b = 0; b < NB_; b++) acc[i][b] = mfma(as_bf(av[u][i][q]), fb[b][q], acc[i][b]);
        }
    }
}

// Grouped launch: [dW1 tiles: NT1 column tiles x S1 splits][dW2: 4 x S1][dW3: S3 splits].
// dW1[n1][f] = sum_m dh1[m][n1] x[m][f]; dW2[n2][n1] = sum_m dh2[m][n2] h1[m][n1];
// dW3[j][n] = sum_m dz[m][j] h2[m][n]. Each writes fp32 partials [split][rows][cols].
__global__ __launch_bounds__(256) void k_wgrad(D1PPOStep a, Work w) {
    if (!cursor_ok(a)) return;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, lr = lane & 31, lh = lane >> 5;
    const int mb = a.mb, s1 = mb / KW;
    int b = blockIdx.x;
    if (b < NT1 * s1) {
        const int tile = b % NT1, split = b / NT1;
        floatx16 acc[2][2] = {};
        wgrad_tile<2, 2, true, 4>(w.dh1t, H, 64 * wave, w.xt, K1, 64 * tile, mb, split * KW, KW, acc);
        float *out = w.part1 + (size_t)split * H * K1;
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            const int f = 64 * tile + 32 * bb + lr;
            if (f < K1) {
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int r = 0; r < 16; r++) out[(size_t)(64 * wave + 32 * i + drow(r, lh)) * K1 + f] = acc[i][bb][r];
            }
        }
        return;
    }
    b -= NT1 * s1;
    if (b < 4 * s1) {
        const int tile = b % 4, split = b / 4;
        floatx16 acc[2][2] = {};
        wgrad_tile<2, 2, false, 2>(w.dh2t, H, 64 * wave, w.h1t, H, 64 * tile, mb,
                                   split * KW, KW, acc);
        float *out = w.part2 + (size_t)split * H * H;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int bb = 0; bb < 2; bb++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    out[(size_t)(64 * wave + 32 * i + drow(r, lh)) * H + 64 * tile + 32 * bb + lr] = acc[i][bb][r];
        return;
    }
    b -= 4 * s1;
    floatx16 acc[1][2] = {};
    wgrad_tile<1, 2, false, 4>(w.dzt, NZ, 0, w.h2t, H, 64 * wave, mb, b * KW3, KW3, acc);
    float *out = w.part3 + (size_t)b * NZ * H;
#pragma unroll
    for (int bb = 0; bb < 2; bb++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int j = drow(r, lh);
            if (j < NZ) out[(size_t)j * H + 64 * wave + 32 * bb + lr] = acc[0][bb][r];
        }
}

// ---------------------------------------------------------------- k_reduce
__device__ __forceinline__ float block_sum(float x, float *red) {
    red[threadIdx.x] = x;
    __syncthreads();
    for (int o = blockDim.x / 2; o; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    return red[0];
}

__global__ __launch_bounds__(256) void k_reduce(D1PPOStep a, Work w) {
    __shared__ float red[256];
    const bool ok = cursor_ok(a);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        a.cursor[1] = ok ? 1 : 0;   // k_adam reads this instead of the cursor it advances
        if (ok) a.step[1] = a.step[0] + 1.f;
    }
    if (!ok) return;
    const int t = threadIdx.x, mb = a.mb, s1 = mb / KW, s3 = mb / KW3;
    uint16_t *g = (uint16_t *)a.g;
    float sq = 0.f;
    if (blockIdx.x < NRED) {
        constexpr int U1 = H * K1 / 4, U2 = H * H / 4, U3 = NZ * H / 4;
        for (int u = blockIdx.x * 256 + t; u < U1 + U2 + U3; u += NRED * 256) {
            const float *src;
            int S;
            size_t stride;
            uint16_t *dst;
            if (u < U1) {
                src = w.part1 + 4 * (size_t)u, S = s1, stride = (size_t)H * K1, dst = g + a.off_w1 + 4 * (size_t)u;
            } else if (u < U1 + U2) {
                const int e = u - U1;
                src = w.part2 + 4 * e, S = s1, stride = (size_t)H * H, dst = g + a.off_w2 + 4 * e;
            } else {
                const int e = u - U1 - U2;
                src = w.part3 + 4 * e, S = s3, stride = (size_t)NZ * H, dst = g + a.off_w3 + 4 * e;
            }
            float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int q0 = 0; q0 < S; q0 += 8) {   // eight loads in flight, summed in split order
                float4 x[8];
#pragma unroll
                for (int j = 0; j < 8; j++)
                    x[j] = q0 + j < S ? *(const float4 *)(src + (q0 + j) * stride) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int j = 0; j < 8; j++) s.x += x[j].x, s.y += x[j].y, s.z += x[j].z, s.w += x[j].w;
            }
            const uint16_t h0 = rb(s.x), h1 = rb(s.y), h2 = rb(s.z), h3 = rb(s.w);
            *(uint2 *)dst = make_uint2((uint32_t)h0 | ((uint32_t)h1 << 16), (uint32_t)h2 | ((uint32_t)h3 << 16));
            sq += bf(h0) * bf(h0) + bf(h1) * bf(h1) + bf(h2) * bf(h2) + bf(h3) * bf(h3);
        }
    } else {   // biases: 64 columns per workgroup, 4 lanes per column over the row partials
        const int col = 64 * (blockIdx.x - NRED) + (t & 63), part = t >> 6, nrows = mb / R;
        float s = 0.f;
        if (col < 2 * H + NZ)
            for (int r0 = part; r0 < nrows; r0 += 32) {   // eight loads in flight
                float x[8];
#pragma unroll
                for (int j = 0; j < 8; j++) x[j] = r0 + 4 * j < nrows ? w.bpart[(size_t)(r0 + 4 * j) * BP + col] : 0.f;
#pragma unroll
                for (int j = 0; j < 8; j++) s += x[j];
            }
        red[t] = s;
        __syncthreads();
        if (t < 64 && col < 2 * H + NZ) {
            const uint16_t hb = rb(red[t] + red[t + 64] + red[t + 128] + red[t + 192]);
            uint16_t *dst = col < H ? g + a.off_b1 + col : col < 2 * H ? g + a.off_b2 + (col - H) : g + a.off_b3 + (col - 2 * H);
            *dst = hb;
            sq = bf(hb) * bf(hb);
        }
        __syncthreads();
    }
    const float tot = block_sum(sq, red);
    if (t == 0) w.npart[blockIdx.x] = tot;
}

// ---------------------------------------------------------------- k_adam
// Global-norm clip + Adam (torch.optim.Adam, no weight decay) over the flat buffers. Every
// workgroup re-sums the norm partials; t = step[1] (set by k_reduce); workgroup 0 stores it
// back to step[0] and advances the minibatch cursor.
__global__ __launch_bounds__(256) void k_adam(D1PPOStep a, Work w) {
    __shared__ float red[256];
    if (a.cursor[1] == 0) return;
    float acc = 0.f;
    for (int j = threadIdx.x; j < NRED + NBIASB; j += blockDim.x) acc += w.npart[j];
    const float norm = sqrtf(block_sum(acc, red));
    const float coef = fminf(a.max_grad_norm / (norm + 1e-6f), 1.f);
    const float tt = a.step[1];
    const float bc1 = 1.f - powf(a.beta1, tt), bc2 = 1.f - powf(a.beta2, tt);
    const float step_size = a.lr / bc1, bc2s = sqrtf(bc2);
    const uint16_t *g = (const uint16_t *)a.g;
    uint16_t *pb = (uint16_t *)a.pb, *w2t = (uint16_t *)a.w2t, *w3t = (uint16_t *)a.w3t;
    for (int64_t i4 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; 4 * i4 < a.nparams;
         i4 += (int64_t)gridDim.x * blockDim.x) {   // four parameters per lane
        const int64_t i0 = 4 * i4;
        const uint2 gv = *(const uint2 *)(g + i0);
        float4 pv = *(const float4 *)(a.p + i0), mv = *(const float4 *)(a.m + i0), vv = *(const float4 *)(a.v + i0);
        const float gs[4] = {bf((uint16_t)gv.x), bf((uint16_t)(gv.x >> 16)), bf((uint16_t)gv.y), bf((uint16_t)(gv.y >> 16))};
        float *pp = &pv.x, *mm = &mv.x, *vq = &vv.x;
        uint16_t h[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float gi = gs[e] * coef;
            mm[e] = a.beta1 * mm[e] + (1.f - a.beta1) * gi;
            vq[e] = a.beta2 * vq[e] + (1.f - a.beta2) * gi * gi;
            pp[e] = pp[e] - step_size * mm[e] / (sqrtf(vq[e]) / bc2s + a.eps);
            h[e] = rb(pp[e]);
        }
        *(float4 *)(a.p + i0) = pv;
        *(float4 *)(a.m + i0) = mv;
        *(float4 *)(a.v + i0) = vv;
        *(uint2 *)(pb + i0) = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int64_t e2 = i0 + e - a.off_w2, e3 = i0 + e - a.off_w3;
            if (e2 >= 0 && e2 < H * H) w2t[(e2 & (H - 1)) * H + (e2 >> 8)] = h[e];
            if (e3 >= 0 && e3 < NZ * H) w3t[(e3 & (H - 1)) * 32 + (e3 >> 8)] = h[e];
        }
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        a.step[0] = tt;
        a.cursor[0] += 1;
    }
}

struct Layout {
    size_t h1t, h2t, dh2t, dh1t, dzt, xt, bpart, part1, part2, part3, npart, total;
};
static Layout layout(int mb) {
    Layout L{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += (bytes + 255) / 256 * 256;
        return at;
    };
    const size_t s1 = (size_t)mb / KW, s3 = (size_t)mb / KW3;
    L.h1t = take((size_t)H * mb * 2);
    L.h2t = take((size_t)H * mb * 2);
    L.dh2t = take((size_t)H * mb * 2);
    L.dh1t = take((size_t)H * mb * 2);
    L.dzt = take((size_t)NZ * mb * 2);
    L.xt = take((size_t)K1 * mb);
    L.bpart = take((size_t)(mb / R) * BP * 4);
    L.part1 = take(s1 * H * K1 * 4);
    L.part2 = take(s1 * H * H * 4);
    L.part3 = take(s3 * NZ * H * 4);
    L.npart = take((size_t)(NRED + NBIASB) * 4);
    L.total = off;
    return L;
}

}  // namespace d1q

extern "C" int64_t d1_ppo_work_bytes(int mb) {
    if (mb <= 0 || mb % d1q::KW) return D1_E_ARG;
    return (int64_t)d1q::layout(mb).total;
}

extern "C" int d1_ppo_step(const D1PPOStep *s, void *stream) {
    using namespace d1q;
    if (!s) return D1_E_ARG;
    const D1PPOStep &a = *s;
    if (a.mb <= 0 || a.mb % KW || a.n < a.mb || a.n >= ((int64_t)1 << 31) || a.nparams % 4) return D1_E_ARG;
    if (!a.obs || !a.perm || !a.cursor || !a.actions || !a.logp_old || !a.adv || !a.ret || !a.p || !a.pb || !a.g ||
        !a.m || !a.v || !a.w2t || !a.w3t || !a.step || !a.loss_parts || !a.work)
        return D1_E_ARG;
    if ((uintptr_t)a.obs % 8 || (uintptr_t)a.pb % 16 || (uintptr_t)a.g % 16 || (uintptr_t)a.w2t % 16 ||
        (uintptr_t)a.w3t % 16 || (uintptr_t)a.work % 256 || (uintptr_t)a.p % 16 || (uintptr_t)a.m % 16 ||
        (uintptr_t)a.v % 16)
        return D1_E_ARG;
    const int64_t offs[6] = {a.off_w1, a.off_b1, a.off_w2, a.off_b2, a.off_w3, a.off_b3};
    const int64_t sizes[6] = {(int64_t)H * K1, H, (int64_t)H * H, H, (int64_t)NZ * H, NZ};
    for (int i = 0; i < 6; i++)
        if (offs[i] < 0 || offs[i] % 8 || offs[i] + sizes[i] > a.nparams) return D1_E_ARG;
    const Layout L = layout(a.mb);
    if (a.work_bytes < (int64_t)L.total) return D1_E_ARG;
    char *base = (char *)a.work;
    Work w;
    w.h1t = (uint16_t *)(base + L.h1t);
    w.h2t = (uint16_t *)(base + L.h2t);
    w.dh2t = (uint16_t *)(base + L.dh2t);
    w.dh1t = (uint16_t *)(base + L.dh1t);
    w.dzt = (uint16_t *)(base + L.dzt);
    w.xt = (uint8_t *)(base + L.xt);
    w.bpart = (float *)(base + L.bpart);
    w.part1 = (float *)(base + L.part1);
    w.part2 = (float *)(base + L.part2);
    w.part3 = (float *)(base + L.part3);
    w.npart = (float *)(base + L.npart);
    const int s1 = a.mb / KW, s3 = a.mb / KW3;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(k_rows, dim3(a.mb / R), dim3(512), 0, st, a, w);
    hipLaunchKernelGGL(k_wgrad, dim3(NT1 * s1 + 4 * s1 + s3), dim3(256), 0, st, a, w);
    hipLaunchKernelGGL(k_reduce, dim3(NRED + NBIASB), dim3(256), 0, st, a, w);
    const int64_t nadam = (a.nparams / 4 + 255) / 256;
    hipLaunchKernelGGL(k_adam, dim3((unsigned)(nadam < NADAM ? nadam : NADAM)), dim3(256), 0, st, a, w);
    return (int)hipGetLastError();
}
