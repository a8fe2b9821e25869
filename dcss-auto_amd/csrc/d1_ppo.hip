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
//             LDS, and leave for the weight gradients in fragment order (below).
//   k_wgrad   dW1 = dh1^T x, dW2 = dh2^T h1, dW3 = dz^T h2 in one grouped launch of split-K
//             MFMA tiles with fp32 partials.
//   k_reduce  fixed-order sums of the partials -> bf16 gradients (one rounding, as the bf16
//             GEMM gives), and sum-of-squares partials for the clipping norm.
//   k_adam    global-norm clip + Adam on the fp32 masters, the bf16 copy, the fragment-ordered
//             weight copies the next k_rows reads, and the minibatch cursor.
//
// MFMA operand layouts, the K order inside a chunk and the fragment order are those of
// d1_frag.h. The weights are kept in fragment order by k_adam (and d1_ppo_prepare), the
// activations and gradients by k_rows; the uint8 x copy uses 16-byte pieces (two per lane
// and chunk).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/d1hip.h"
#include "d1_frag.h"

namespace d1q {

using namespace d1f;

constexpr int K1 = 1800;              // observation bytes = layer-1 inputs
constexpr int H = 256;                // hidden width
constexpr int NA = 16, NZ = 17;       // logits, head width
constexpr int R = 32;                 // samples per k_rows workgroup
constexpr int XS = H + 8;             // LDS row stride (bf16) of the [32][256] activation tiles
constexpr int DS = 40;                // LDS row stride (bf16) of the dz tile (32 columns used)
constexpr int XR = K1 + 16;           // LDS row stride (bf16) of k_rows' x tile: 908 dwords, so the
                                      // 16-byte fragment reads of 16 consecutive rows hit distinct banks
constexpr int BP = 544;               // bias partial row: db1[256] | db2[256] | db3[17] | loss sum | pad
constexpr int C1 = 29;                // layer-1 K chunks (28 of 64 + the 8 inputs 1792..1799)
constexpr int XB = 57;                // 32-row blocks of the x copy (1824 rows, 1800..1823 zero)
constexpr int KW = 1024;              // samples per dW1 / dW2 workgroup
constexpr int KW3 = 256;              // samples per dW3 / dW1-tail slice (one workgroup each)
constexpr int NT1 = 28;               // dW1 column tiles of 64 (inputs 0..1791; 1792..1799 are the tail)
constexpr int NRF = (H * NT1 * 64 + H * H) / 4 / 256;   // k_reduce workgroups of mb/KW-partial units (dW1 columns
                                                       // < 1792, dW2), one unit of four elements per lane
constexpr int NRS = (H * 2 + NZ * H / 4) * 4 / 256;    // k_reduce workgroups of mb/KW3-partial units (dW1 columns
                                                       // 1792..1799, dW3), four lanes per unit
constexpr int NRED = NRF + NRS;
static_assert((H * NT1 * 64 + H * H) % 1024 == 0 && (H * 2 + NZ * H / 4) * 4 % 256 == 0, "k_reduce unit split");
constexpr int NBIASB = (2 * H + NZ + 7) / 8;     // k_reduce bias workgroups (8 columns x 32 lanes each)

// packed weight copies (bf16 elements), all in fragment order
constexpr int P_W1 = 0;                          // layer 1 B (W1 rows): [8 blocks][29 chunks][4][64][8]
constexpr int P_W2 = P_W1 + 8 * C1 * 4 * 512;    // layer 2 B (W2 rows): [8][4][4][64][8]
constexpr int P_W2T = P_W2 + 8 * 4 * 4 * 512;    // dh1 B (W2 columns): [8][4][4][64][8]
constexpr int P_W3 = P_W2T + 8 * 4 * 4 * 512;    // head B (W3 rows, 17 of 32 lanes): [8][2][64][8]
constexpr int P_W3T = P_W3 + 8 * 2 * 512;        // dh2 B (W3 columns, k < 17): [8][2][64][8]
constexpr int P_END = P_W3T + 8 * 2 * 512;

struct Work {
    uint16_t *wpk;                       // packed weights (state kept between calls)
    uint16_t *h1f, *h2f, *dh2f, *dh1f;   // [256 rows][mb] bf16, fragment order
    uint16_t *dzf;                       // [32 rows (17 used)][mb] bf16, fragment order
    uint8_t *xf;                         // [1824 rows][mb] uint8 x^T, 16-byte fragment order
    float *bpart;                        // [mb/32][BP]
    float *part1, *part2, *part3;        // [mb/KW][256][1800] (columns < 1792), [mb/KW][256][256], [mb/KW3][17][256]
    float *part1t;                       // [mb/KW3][256][8]: dW1 columns 1792..1799
    float *npart;                        // [NRED + NBIASB] sum-of-squares partials
};

__device__ __forceinline__ int64_t clamp_index(int64_t s, int64_t n) { return s < 0 ? 0 : (s >= n ? n - 1 : s); }
// The cursor is read with a vector load (an agent-scope relaxed atomic load): a scalar load
// is waited for together with the kernel-argument loads (scalar loads return out of order),
// so every later instruction would wait for the cursor's round trip.
__device__ __forceinline__ int load_cursor(const int32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool cursor_ok(const D1PPOStep &a, int cur) { return cur >= 0 && (int64_t)(cur + 1) * a.mb <= a.n; }
__device__ __forceinline__ bool cursor_ok(const D1PPOStep &a) { return cursor_ok(a, load_cursor(a.cursor)); }
// A cursor value `cur` (loaded early) made to depend on `after` (an empty asm): the check on
// it, and the wait for its load, then come after the loads that produce `after`, which so
// do not wait for the cursor's round trip.
__device__ __forceinline__ int after(int cur, float after) {
    asm volatile("" : "+v"(cur) : "v"(after));
    return cur;
}
// fragment order for the uint8 x copy: 16-byte pieces, two per lane and chunk
__device__ __forceinline__ size_t xidx(int row, int k, int nch) {
    return ((((size_t)(row >> 5) * nch + (k >> 6)) * 2 + ((k >> 4) & 1)) * 64 + (row & 31) + 32 * ((k >> 5) & 1)) * 16 +
           (k & 15);
}
// packed-weight slots of each parameter element
__device__ __forceinline__ int pk_w1(int n, int k) { return P_W1 + (int)fidx(n, k, C1); }     // W1[n][k]
__device__ __forceinline__ int pk_w2(int n, int k) { return P_W2 + (int)fidx(n, k, 4); }      // W2[n][k]
__device__ __forceinline__ int pk_w2t(int o, int i) { return P_W2T + (int)fidx(i, o, 4); }    // W2[o][i] as B[o][i]
__device__ __forceinline__ int pk_w3(int j, int k) {   // head: wave k/32 contracts k = 32w + 16s + 8h + jj
    return P_W3 + (((k >> 5) * 2 + ((k >> 4) & 1)) * 64 + j + 32 * ((k >> 3) & 1)) * 8 + (k & 7);
}
__device__ __forceinline__ int pk_w3t(int j, int c) {  // dh2: slot 8h + jj of step s is k = j = 16s + 8h + jj
    return P_W3T + (((c >> 5) * 2 + (j >> 4)) * 64 + (c & 31) + 32 * ((j >> 3) & 1)) * 8 + (j & 7);
}
// one fragment (16 bytes per lane) of a packed operand
__device__ __forceinline__ bf16x8 frag(const uint16_t *base, int idx, int lane) {
    return as_bf(*(const uint4 *)(base + ((size_t)idx * 64 + lane) * 8));
}

// ---------------------------------------------------------------- k_rows
// Epilogue shared by the four row-block products: v[r] (fp32, this lane's column c) ->
// bf16 bits, LDS row-major tile (if any), the fragment-ordered global copy (rows = columns
// c, k = samples), bit r of *mask set where the bf16 value is > 0 (if asked), and the column
// sum of the bf16 values (lanes < 32 hold the full 32-row sum afterwards).
__device__ __forceinline__ float rows_out(const float (&v)[16], uint16_t *tile, uint16_t *gf, int nch, int m0, int c,
                                          int lh, uint32_t *mask) {
    uint16_t hb[16];
    float colsum = 0.f;
    uint32_t pos = 0;
#pragma unroll
    for (int r = 0; r < 16; r += 2) {   // hardware pack, two values per instruction
        const uint32_t w2 = cvt2(v[r], v[r + 1]);
        hb[r] = (uint16_t)(w2 & 0xFFFFu);
        hb[r + 1] = (uint16_t)(w2 >> 16);
    }
#pragma unroll
    for (int r = 0; r < 16; r++) {
        colsum += bf(hb[r]);
        if (bf(hb[r]) > 0.f) pos |= 1u << r;
        if (tile) tile[drow(r, lh) * XS + c] = hb[r];
    }
    if (mask) *mask = pos;
#pragma unroll
    for (int g = 0; g < 4; g++)   // samples m0 + 8g + 4h .. +3 are registers 4g .. 4g+3
        *(uint2 *)(gf + fidx(c, m0 + 8 * g + 4 * lh, nch)) =
            make_uint2((uint32_t)hb[4 * g] | ((uint32_t)hb[4 * g + 1] << 16),
                       (uint32_t)hb[4 * g + 2] | ((uint32_t)hb[4 * g + 3] << 16));
    return xor32_sum(colsum);
}

__global__ __launch_bounds__(512) void k_rows(D1PPOStep a, Work w) {
    // The 32 x rows, widened once to bf16 (116 KB of the CU's 160 KB), share their LDS with
    // the tiles of the later phases.
    __shared__ __align__(16) uint8_t lds[R * XR * 2];
    uint16_t *xs = (uint16_t *)lds;                                          // x rows (bf16), stride XR
    uint16_t *x1 = (uint16_t *)lds;                                          // h1, later dh2 (row-major)
    uint16_t *x2 = (uint16_t *)(lds + R * XS * 2);                           // h2
    uint16_t *dzs = (uint16_t *)(lds + 2 * R * XS * 2);                      // dL/dz, columns 17..31 zero
    float(*zp)[R][NZ] = (float(*)[R][NZ])(lds + 2 * R * XS * 2 + R * DS * 2);   // head partials per wave
    static_assert(2 * R * XS * 2 + R * DS * 2 + 8 * R * NZ * 4 <= R * XR * 2, "LDS union");
    __shared__ int64_t soff[R];   // byte offset of each sample's observation row
    __shared__ float sold[R], sadv[R], sret[R];
    __shared__ int sact[R];
    __shared__ float lsum[8][3];
    __shared__ float dzsum[8][NZ];
    if (!cursor_ok(a)) return;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, lr = lane & 31, lh = lane >> 5;
    const int mb = a.mb, nch = mb / 64, m0 = blockIdx.x * R;
    const int64_t base = (int64_t)a.cursor[0] * mb + m0;
    const uint16_t *pb = (const uint16_t *)a.pb;
    const uint16_t *B1 = pb + a.off_b1, *B2 = pb + a.off_b2, *B3 = pb + a.off_b3;
    const uint16_t *wpk = w.wpk;
    const int c = 32 * wave + lr;   // this lane's column in every layer

    // layer-1 weights: 4-deep ring of fragment-ordered chunks, the first three issued now
    uint4 wb[4][4];
    auto wload = [&](uint4 (&dst)[4], int ch) {
#pragma unroll
        for (int q = 0; q < 4; q++) dst[q] = *(const uint4 *)(wpk + P_W1 + ((size_t)((wave * C1 + ch) * 4 + q) * 64 + lane) * 8);
    };
    wload(wb[0], 0);
    wload(wb[1], 1);
    wload(wb[2], 2);
    // the small operands of the later phases (biases, head weights), loaded now: the previous
    // step's update wrote them from other XCDs, and loaded where they are used their latency
    // was waited out in full at each phase
    const uint16_t b1c = B1[c], b2c = B2[c], b3j = B3[t & 15], b3v = B3[NA];
    const bf16x8 w3f0 = frag(wpk + P_W3, wave * 2, lane), w3f1 = frag(wpk + P_W3, wave * 2 + 1, lane);
    const bf16x8 w3t0 = frag(wpk + P_W3T, wave * 2, lane), w3t1 = frag(wpk + P_W3T, wave * 2 + 1, lane);
    // the sample rows: their observation offsets go to LDS first, so that the row loads below
    // wait for one load level only; the per-sample scalars are loaded after the rows and
    // reach LDS at the barrier halfway through layer 1 (the loss reads them much later)
    int64_t srow = 0;
    if (t < R) {
        srow = clamp_index(a.perm[base + t], a.n);   // entries outside [0, n) are a caller error
        soff[t] = srow * K1;
    }
    __syncthreads();
    // The 32 observation rows, in units of 16 rows x 4 inputs: widened to bf16 into the LDS
    // tile, and transposed in registers into the x^T copy for the dW1 product, one 16-byte
    // piece per input (rows 1800..1823 of the copy are written as zeros). Inputs 0..895
    // (chunks 0..13) are stored first; the loads of the rest are in flight meanwhile and are
    // stored once layer 1 reaches chunk 14, so the gather overlaps the weight stream.
    constexpr int KA = 224, KBN = K1 / 4 - KA;   // 4-input groups of each half
    uint32_t xa[16], xb[16];
    const int ua = min(t, 2 * KA - 1), pa = ua / KA, ka = ua - pa * KA;
    const int ub = min(t, 2 * KBN - 1), pbb = ub / KBN, kb = KA + ub - pbb * KBN;
#pragma unroll
    for (int j = 0; j < 16; j++) xa[j] = *(const uint32_t *)(a.obs + soff[16 * pa + j] + 4 * ka);   // unconditional:
#pragma unroll
    for (int j = 0; j < 16; j++) xb[j] = *(const uint32_t *)(a.obs + soff[16 * pbb + j] + 4 * kb);  // spare lanes repeat
    int sa = 0;
    float so = 0.f, sd = 0.f, sr = 0.f;
    if (t < R) {
        sa = (int)a.actions[srow];
        so = a.logp_old[srow];
        sd = a.adv[srow];
        sr = a.ret[srow];
    }
    auto xstore = [&](const uint32_t (&x)[16], int p, int kg) {
#pragma unroll
        for (int j = 0; j < 16; j++) *(uint2 *)(xs + (16 * p + j) * XR + 4 * kg) = widen4(x[j]);
        // 4x4 byte transposes with v_perm: o[e][d] = byte e of samples 4d..4d+3
        uint32_t o[4][4];
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const uint32_t *y = &x[4 * d];
            const uint32_t a01 = __builtin_amdgcn_perm(y[1], y[0], 0x05010400u);   // y0.0 y1.0 y0.1 y1.1
            const uint32_t b01 = __builtin_amdgcn_perm(y[1], y[0], 0x07030602u);   // y0.2 y1.2 y0.3 y1.3
            const uint32_t a23 = __builtin_amdgcn_perm(y[3], y[2], 0x05010400u);
            const uint32_t b23 = __builtin_amdgcn_perm(y[3], y[2], 0x07030602u);
            o[0][d] = __builtin_amdgcn_perm(a23, a01, 0x05040100u);
            o[1][d] = __builtin_amdgcn_perm(a23, a01, 0x07060302u);
            o[2][d] = __builtin_amdgcn_perm(b23, b01, 0x05040100u);
            o[3][d] = __builtin_amdgcn_perm(b23, b01, 0x07060302u);
        }
#pragma unroll
        for (int e = 0; e < 4; e++)
            *(uint4 *)(w.xf + xidx(4 * kg + e, m0 + 16 * p, nch)) = make_uint4(o[e][0], o[e][1], o[e][2], o[e][3]);
    };
    if (t < 2 * KA) xstore(xa, pa, ka);
    if (t < 2 * (XB * 32 - K1))
        *(uint4 *)(w.xf + xidx(K1 + (t >> 1), m0 + 16 * (t & 1), nch)) = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
    float v[16];

    // ---- layer 1: 28 chunks of 64 inputs (A from the LDS rows, W1 from the ring, loads
    // issued 3 chunks ahead), then chunk 28 = inputs 1792..1799 (lower half, q = 0)
    uint32_t mask1 = 0, mask2 = 0;
    bf16x8 w2f[16];   // layer-2 weight fragments (chunk ch, step q at 4 ch + q), then dh1's
    {
        const uint16_t *xr = xs + lr * XR + 32 * lh;
        floatx16 e0 = {}, e1 = {};
        for (int i0 = 0; i0 < 28; i0 += 4) {
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int ch = i0 + u;
                if (ch == 14) {   // the second half of the x rows and the sample scalars (uniform branch)
                    if (t < 2 * KBN) xstore(xb, pbb, kb);
                    if (t < R) sact[t] = sa, sold[t] = so, sadv[t] = sd, sret[t] = sr;
                    __syncthreads();
                }
                if (ch + 3 < C1) wload(wb[(u + 3) & 3], ch + 3);
                e0 = mfma(as_bf(*(const uint4 *)(xr + 64 * ch)), as_bf(wb[u][0]), e0);
                e1 = mfma(as_bf(*(const uint4 *)(xr + 64 * ch + 8)), as_bf(wb[u][1]), e1);
                e0 = mfma(as_bf(*(const uint4 *)(xr + 64 * ch + 16)), as_bf(wb[u][2]), e0);
                e1 = mfma(as_bf(*(const uint4 *)(xr + 64 * ch + 24)), as_bf(wb[u][3]), e1);
            }
        }
        // chunk 28 sits in ring slot 0 (loaded during chunk 25); its slots past input 1799 hold zeros
        const uint4 xt = lh == 0 ? *(const uint4 *)(xs + lr * XR + 1792) : make_uint4(0u, 0u, 0u, 0u);
        e0 = mfma(as_bf(xt), as_bf(wb[0][0]), e0);
#pragma unroll
        for (int q = 0; q < 16; q++) w2f[q] = frag(wpk + P_W2, wave * 16 + q, lane);   // layer 2's weights
        __syncthreads();   // every wave is done with the x rows before h1 overwrites them
        const float bias = bf(b1c);
#pragma unroll
        for (int r = 0; r < 16; r++) v[r] = fmaxf(e0[r] + e1[r] + bias, 0.f);
        rows_out(v, x1, w.h1f, nch, m0, c, lh, &mask1);
    }
    __syncthreads();

    // ---- layer 2: h2 = relu(h1 W2^T + b2), K = 256 from the LDS h1 tile
    {
        const uint16_t *ar = x1 + lr * XS + 32 * lh;
        floatx16 e0 = {}, e1 = {};
#pragma unroll
        for (int ch = 0; ch < 4; ch++) {
            bf16x8 fa[4], fb[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                fa[q] = as_bf(*(const uint4 *)(ar + 64 * ch + 8 * q));
                fb[q] = w2f[4 * ch + q];
            }
            e0 = mfma(fa[0], fb[0], e0);
            e1 = mfma(fa[1], fb[1], e1);
            e0 = mfma(fa[2], fb[2], e0);
            e1 = mfma(fa[3], fb[3], e1);
        }
#pragma unroll
        for (int q = 0; q < 16; q++) w2f[q] = frag(wpk + P_W2T, wave * 16 + q, lane);   // dh1's weights
        const float bias = bf(b2c);
#pragma unroll
        for (int r = 0; r < 16; r++) v[r] = fmaxf(e0[r] + e1[r] + bias, 0.f);
        rows_out(v, x2, w.h2f, nch, m0, c, lh, &mask2);
    }
    __syncthreads();

    // ---- head partials: wave w contracts k = 32w..32w+31 (two K16 steps, slot 8h+j <-> k = 32w+16s+8h+j)
    {
        floatx16 zacc = {};
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const uint4 av = *(const uint4 *)(x2 + lr * XS + 32 * wave + 16 * s + 8 * lh);
            zacc = mfma(as_bf(av), s ? w3f1 : w3f0, zacc);
        }
        if (lr < NZ) {
#pragma unroll
            for (int r = 0; r < 16; r++) zp[wave][drow(r, lh)][lr] = zacc[r];
        }
    }
    __syncthreads();

    // ---- loss and dL/dz: 16 lanes per sample (lane j = logit j; lane 0 also the value)
    {
        const int r = t >> 4, j = t & 15;
        float zj = zp[0][r][j], zv = zp[0][r][NA];
#pragma unroll
        for (int q = 1; q < 8; q++) zj += zp[q][r][j], zv += zp[q][r][NA];
        const float l = bf(rb(zj + bf(b3j)));         // the head output is bf16
        const float value = bf(rb(zv + bf(b3v)));
        if (a.z_out) {
            a.z_out[(size_t)(m0 + r) * NZ + j] = l;
            if (j == 0) a.z_out[(size_t)(m0 + r) * NZ + NA] = value;
        }
        const float mx = row16_max(l);   // reductions over the sample's 16 lanes
        const float se = row16_sum(expf(l - mx));
        const float ls = logf(se);
        const float lp = l - mx - ls, p = expf(lp);
        const int act = sact[r];
        const float hh = row16_sum(-p * lp), la = row16_sum(j == act ? l : 0.f);
        const float lpa = la - mx - ls;
        const float ratio = expf(lpa - sold[r]);
        const float A = sadv[r];
        const float un = ratio * A, cl = fminf(fmaxf(ratio, 1.f - a.clip), 1.f + a.clip) * A;
        const float gr = un <= cl ? -A : 0.f;   // torch.minimum routes ties to its first argument
        const float d = value - sret[r];
        const float inv = 1.f / (float)mb;
        const uint16_t dzj = rb((gr * ratio * ((j == act ? 1.f : 0.f) - p) + a.ecoef * p * (lp + hh)) * inv);
        dzs[r * DS + j] = dzj;
        dzs[r * DS + NZ + j] = 0;   // columns 17..32 (32 is padding)
        w.dzf[fidx(j, m0 + r, nch)] = dzj;
        if (j == 0) {
            const uint16_t dzv = rb(a.vcoef * d * inv);
            dzs[r * DS + NA] = dzv;
            w.dzf[fidx(NA, m0 + r, nch)] = dzv;
        }
        // column sums of dz over this wave's 4 samples (lanes j, j+16, j+32, j+48)
        float cj = bf(dzj), cv = j == 0 ? bf(rb(a.vcoef * d * inv)) : 0.f;
        cj = xor16_sum(xor32_sum(cj));
        cv = xor16_sum(xor32_sum(cv));
        if (lane < 16) dzsum[wave][j] = cj;
        if (lane == 0) dzsum[wave][NA] = cv;
        // per-sample loss terms (every lane of a group holds them): lane j == 0 of each group
        float pg = j == 0 ? -fminf(un, cl) : 0.f, vl = j == 0 ? 0.5f * d * d : 0.f, ent = j == 0 ? hh : 0.f;
        pg = xor16_sum(xor32_sum(pg));
        vl = xor16_sum(xor32_sum(vl));
        ent = xor16_sum(xor32_sum(ent));
        if (lane == 0) lsum[wave][0] = pg, lsum[wave][1] = vl, lsum[wave][2] = ent;
    }
    __syncthreads();
    if (t < 4) {
        float s = 0.f;
        if (t < 3)
            for (int q = 0; q < 8; q++) s += lsum[q][t];
        a.loss_parts[(size_t)blockIdx.x * 4 + t] = s;
        // the three loss sums also go to the bias-partial row's column 2H+NZ (k_reduce folds
        // their finiteness into the gradient norm)
        float z = s;
        z += dpp_f<DPP_XOR1>(z);
        z += dpp_f<DPP_XOR2>(z);
        if (t == 0) w.bpart[(size_t)blockIdx.x * BP + 2 * H + NZ] = z;
    } else if (t >= 64 && t < 64 + NZ) {   // head-bias partial: the 8 waves' sums
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < 8; q++) s += dzsum[q][t - 64];
        w.bpart[(size_t)blockIdx.x * BP + 2 * H + (t - 64)] = s;
    }

    // ---- dh2 = (dz W3)[h2 > 0]: K = 17 padded to 32, B = W3 columns
    {
        floatx16 acc = {};
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const uint4 av = *(const uint4 *)(dzs + lr * DS + 16 * s + 8 * lh);
            acc = mfma(as_bf(av), s ? w3t1 : w3t0, acc);
        }
#pragma unroll
        for (int r = 0; r < 16; r++) v[r] = (mask2 >> r) & 1u ? acc[r] : 0.f;
        const float cs = rows_out(v, x1, w.dh2f, nch, m0, c, lh, nullptr);
        if (lh == 0) w.bpart[(size_t)blockIdx.x * BP + H + c] = cs;
    }
    __syncthreads();

    // ---- dh1 = (dh2 W2)[h1 > 0]: K = 256 from the LDS dh2 tile, B = W2 columns
    {
        const uint16_t *ar = x1 + lr * XS + 32 * lh;
        floatx16 e0 = {}, e1 = {};
#pragma unroll
        for (int ch = 0; ch < 4; ch++) {
            bf16x8 fa[4], fb[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                fa[q] = as_bf(*(const uint4 *)(ar + 64 * ch + 8 * q));
                fb[q] = w2f[4 * ch + q];
            }
            e0 = mfma(fa[0], fb[0], e0);
            e1 = mfma(fa[1], fb[1], e1);
            e0 = mfma(fa[2], fb[2], e0);
            e1 = mfma(fa[3], fb[3], e1);
        }
#pragma unroll
        for (int r = 0; r < 16; r++) v[r] = (mask1 >> r) & 1u ? e0[r] + e1[r] : 0.f;
        const float cs = rows_out(v, nullptr, w.dh1f, nch, m0, c, lh, nullptr);
        if (lh == 0) w.bpart[(size_t)blockIdx.x * BP + c] = cs;
    }
}

// ---------------------------------------------------------------- k_wgrad
// One split-K tile of out[i][j] = sum_m at[i][m] bt[j][m] over the sample chunks
// [c0, c0 + nc): both operands fragment-ordered with `nch` chunks; `at` bf16, `bt` bf16 or
// (XB_) the uint8 x copy. Wave w owns NA_ row blocks of 32 from row block ib, the workgroup
// NB_ column blocks from jb. Loads run through a RING-deep register ring (issued RING-1
// chunks ahead).
template <int NA_, int NB_, bool XB_, int RING>
__device__ __forceinline__ void wgrad_tile(const uint16_t *at, int ib, int an, const void *bt, int jb, int bn, int nch,
                                           int c0, int nc, floatx16 (&acc)[NA_][NB_]) {
    constexpr int BW = XB_ ? 2 : 4;   // 16-byte pieces per B row block and chunk
    const int lane = threadIdx.x & 63, lr = lane & 31;
    // Row / column blocks past an / bn are read from the last block (in bounds): like the
    // unwritten rows of a block, they only feed outputs that the caller never stores.
    uint4 av[RING][NA_][4], bv[RING][NB_][BW];
    auto load = [&](int slot, int ch) {
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int i = 0; i < NA_; i++)
                av[slot][i][q] = *(const uint4 *)(at + ((((size_t)min(ib + i, an - 1) * nch + ch) * 4 + q) * 64 + lane) * 8);
#pragma unroll
        for (int p = 0; p < BW; p++)
#pragma unroll
            for (int b = 0; b < NB_; b++) {
                const size_t piece = (((size_t)min(jb + b, bn - 1) * nch + ch) * BW + p) * 64 + lane;
                bv[slot][b][p] = XB_ ? *(const uint4 *)((const uint8_t *)bt + piece * 16)
                                     : *(const uint4 *)((const uint16_t *)bt + piece * 8);
            }
    };
#pragma unroll
    for (int u = 0; u + 1 < RING; u++)
        if (u < nc) load(u, c0 + u);
#pragma unroll 1
    for (int k0 = 0; k0 < nc; k0 += RING) {
#pragma unroll
        for (int u = 0; u < RING; u++) {
            const int k = k0 + u;
            if (k < nc) {
                if (k + RING - 1 < nc) load((u + RING - 1) % RING, c0 + k + RING - 1);
                bf16x8 fb[NB_][4];
#pragma unroll
                for (int b = 0; b < NB_; b++) {
                    if (XB_) {
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
}

// The dW1 / dW2 tile: wave w owns A row blocks 2w, 2w+1 (64 rows of `at`), and the four
// waves share column blocks jb, jb+1 of `bt`. The shared B chunk is loaded once per
// workgroup (one or two 16-byte pieces per lane; uint8 widened once), staged as fragments
// in a double-buffered LDS tile `bl` ([2][2 blocks][4 steps][64] of 16 bytes) and read by
// all four waves. A and B loads run two chunks ahead through three named register slots
// (chunk c lives in slot c % 3); one barrier per chunk. Column blocks past bn are read
// from block bn-1 (in bounds): they only feed output columns that the caller never stores,
// and the loads stay free of branches.
template <bool XB_>
__device__ __forceinline__ void wgrad_tile2(const uint16_t *at, const void *bt, int jb, int bn, int nch, int c0, int nc,
                                            uint4 *bl, floatx16 (&acc)[2][2]) {
    constexpr int BPL = XB_ ? 1 : 2;   // B pieces per lane and chunk
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int bb = t >> 7, ph = (t >> 6) & 1;    // this lane's B block and half of the four steps
    const int brow = min(jb + bb, bn - 1);
    // per-lane base addresses; chunk ch adds ch * 4 KB (A, bf16) or ch * 2 or 4 KB (B)
    const uint4 *a0 = (const uint4 *)at + (size_t)(2 * wave) * nch * 256 + lane;
    const uint4 *a1 = a0 + (size_t)nch * 256;
    const u32x4 *b0 = (const u32x4 *)bt + ((size_t)brow * nch * (XB_ ? 2 : 4) + (XB_ ? ph : 2 * ph)) * 64 + lane;
    uint4 aS0[2][4], aS1[2][4], aS2[2][4];
    u32x4 bS0[BPL], bS1[BPL], bS2[BPL];
    auto load = [&](uint4 (&av)[2][4], u32x4 (&bv)[BPL], int ch) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            av[0][q] = a0[ch * 256 + q * 64];
            av[1][q] = a1[ch * 256 + q * 64];
        }
#pragma unroll
        for (int e = 0; e < BPL; e++) bv[e] = b0[ch * (XB_ ? 128 : 256) + e * 64];
    };
    auto bstore = [&](const u32x4 (&bv)[BPL], int buf) {   // fragments q = 2ph, 2ph + 1 of block bb
        u32x4 *dst = (u32x4 *)bl + ((buf * 2 + bb) * 4 + 2 * ph) * 64 + lane;
        if (XB_) {
            dst[0] = __builtin_bit_cast(u32x4, widen8(bv[0].x, bv[0].y));
            dst[64] = __builtin_bit_cast(u32x4, widen8(bv[0].z, bv[0].w));
        } else {
            dst[0] = bv[0];
            dst[64] = bv[BPL - 1];
        }
    };
    // chunk k: issue chunk k+2's loads into the slot chunk k-1 used, multiply, stage chunk
    // k+1's B (loaded two chunks ago) into the other LDS buffer
    auto step = [&](const uint4 (&acur)[2][4], uint4 (&anext)[2][4], u32x4 (&bnext)[BPL], const u32x4 (&bstage)[BPL],
                    int k) {
        if (k + 2 < nc) load(anext, bnext, c0 + k + 2);
        const uint4 *src = bl + (k & 1) * 2 * 4 * 64 + lane;
        bf16x8 fb[2][4];
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int q = 0; q < 4; q++) fb[b][q] = as_bf(src[(b * 4 + q) * 64]);
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int b = 0; b < 2; b++) acc[i][b] = mfma(as_bf(acur[i][q]), fb[b][q], acc[i][b]);
        if (k + 1 < nc) bstore(bstage, (k + 1) & 1);
        __syncthreads();
    };
    load(aS0, bS0, c0);
    if (nc > 1) load(aS1, bS1, c0 + 1);
    bstore(bS0, 0);
    __syncthreads();
    for (int k0 = 0; k0 < nc; k0 += 3) {
        step(aS0, aS2, bS2, bS1, k0);
        if (k0 + 1 < nc) step(aS1, aS0, bS0, bS2, k0 + 1);
        if (k0 + 2 < nc) step(aS2, aS1, bS1, bS0, k0 + 2);
    }
}

// Grouped launch of 32 * mb/KW + mb/KW3 workgroups (288 at mb = 8192, up to two per CU):
// [dW1: NT1 column tiles x mb/KW splits][dW2: 4 column tiles x mb/KW splits][mb/KW3 slices
// of dW3 and of the dW1 tail]. The slices had ridden on the dW2 workgroups, which then
// finished last; on their own they run beside the tiles (update 0.2474 -> 0.2434 s at C4). dW1[n1][f] = sum_m dh1[m][n1] x[m][f];
// dW2[n2][n1] = sum_m dh2[m][n2] h1[m][n1]; dW3[j][n] = sum_m dz[m][j] h2[m][n]. Each writes
// fp32 partials [split][rows][cols]. The dW1 splits of one column tile are consecutive
// blocks, which a launch spreads over the eight XCDs, so each XCD's L2 serves one sample
// range of dh1 to every column tile.
__global__ __launch_bounds__(256, 2) void k_wgrad(D1PPOStep a, Work w) {
    __shared__ uint4 bl[2 * 2 * 4 * 64];
    // the cursor is checked before the stores only: the operand loads do not wait for it
    // (past the end of the buffer the tiles multiply stale operands and store nothing)
    const int cur = load_cursor(a.cursor);
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, lr = lane & 31, lh = lane >> 5;
    const int mb = a.mb, nch = mb / 64, s1 = mb / KW;
    int b = blockIdx.x;
    if (b < NT1 * s1) {
        const int tile = b / s1, split = b % s1;
        floatx16 acc[2][2] = {};
        wgrad_tile2<true>(w.dh1f, w.xf, 2 * tile, XB, nch, split * (KW / 64), KW / 64, bl, acc);
        if (!cursor_ok(a, after(cur, acc[0][0][0]))) return;
        float *out = w.part1 + (size_t)split * H * K1;
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            const int f = 64 * tile + 32 * bb + lr;
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) out[(size_t)(64 * wave + 32 * i + drow(r, lh)) * K1 + f] = acc[i][bb][r];
        }
        return;
    }
    b -= NT1 * s1;
    if (b < 4 * s1) {
        const int tile = b / s1, split = b % s1;
        floatx16 acc[2][2] = {};
        wgrad_tile2<false>(w.dh2f, w.h1f, 2 * tile, 8, nch, split * (KW / 64), KW / 64, bl, acc);
        if (!cursor_ok(a, after(cur, acc[0][0][0]))) return;
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
    // slice b of dW3 (wave w: columns 64w..64w+63) and of the dW1 tail (wave w: rows
    // 64w..64w+63 against x^T block 56, inputs 1792..1823, of which 1792..1799 are kept)
    {
        floatx16 acc[1][2] = {};
        wgrad_tile<1, 2, false, 3>(w.dzf, 0, 1, w.h2f, 2 * wave, 8, nch, b * (KW3 / 64), KW3 / 64, acc);
        if (!cursor_ok(a, after(cur, acc[0][0][0]))) return;
        float *out = w.part3 + (size_t)b * NZ * H;
#pragma unroll
        for (int bb = 0; bb < 2; bb++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int j = drow(r, lh);
                if (j < NZ) out[(size_t)j * H + 64 * wave + 32 * bb + lr] = acc[0][bb][r];
            }
    }
    {
        floatx16 acc[2][1] = {};
        wgrad_tile<2, 1, true, 3>(w.dh1f, 2 * wave, 8, w.xf, K1 / 32, XB, nch, b * (KW3 / 64), KW3 / 64, acc);
        float *out = w.part1t + (size_t)b * H * 8;
        if (lr < 8) {
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) out[(size_t)(64 * wave + 32 * i + drow(r, lh)) * 8 + lr] = acc[i][0][r];
        }
    }
}

// ---------------------------------------------------------------- k_reduce
__device__ __forceinline__ float block_sum(float x, float *red) {   // 256 lanes, red[4]
    x = row16_sum(xor16_sum(xor32_sum(x)));   // offsets 32, 16, then 8, 4, 2, 1
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    const float s = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return s;
}

// Sum of S partials (stride apart) of four elements, in partial order, eight loads in flight.
__device__ __forceinline__ float4 sum_parts(const float *src, size_t stride, int S) {
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int q0 = 0; q0 < S; q0 += 8) {
        float4 x[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
            x[j] = q0 + j < S ? *(const float4 *)(src + (q0 + j) * stride) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int j = 0; j < 8; j++) s.x += x[j].x, s.y += x[j].y, s.z += x[j].z, s.w += x[j].w;
    }
    return s;
}
// Four gradient elements -> bf16 at dst; returns the sum of squares of the rounded values.
__device__ __forceinline__ float store_grad4(uint16_t *dst, float4 s) {
    const uint32_t w01 = cvt2(s.x, s.y), w23 = cvt2(s.z, s.w);
    *(uint2 *)dst = make_uint2(w01, w23);
    const float h0 = __uint_as_float(w01 << 16), h1 = __uint_as_float(w01 & 0xFFFF0000u);
    const float h2 = __uint_as_float(w23 << 16), h3 = __uint_as_float(w23 & 0xFFFF0000u);
    return h0 * h0 + h1 * h1 + h2 * h2 + h3 * h3;
}

__global__ __launch_bounds__(256) void k_reduce(D1PPOStep a, Work w) {
    __shared__ float red[256];
    // Past the end of the buffer nothing is stored (the partial loads do not wait for the
    // cursor); workgroup 0 records the decision in cursor[1], which k_adam reads instead of the
    // cursor it advances.
    const int cur = load_cursor(a.cursor);
    auto done = [&](bool ok) {
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            a.cursor[1] = ok ? 1 : 0;
            if (ok) a.step[1] = a.step[0] + 1.f;
        }
    };
    const int t = threadIdx.x, mb = a.mb, s1 = mb / KW;
    uint16_t *g = (uint16_t *)a.g;
    float sq = 0.f;
    if (blockIdx.x < NRF) {   // s1 partials per unit, summed in split order
        const int u = blockIdx.x * 256 + t;
        const float *src;
        size_t stride;
        uint16_t *dst;
        if (u < H * NT1 * 16) {
            const int n = u / (NT1 * 16), f = 4 * (u - n * NT1 * 16);
            src = w.part1 + (size_t)n * K1 + f, stride = (size_t)H * K1, dst = g + a.off_w1 + (size_t)n * K1 + f;
        } else {
            const int e = u - H * NT1 * 16;
            src = w.part2 + 4 * e, stride = (size_t)H * H, dst = g + a.off_w2 + 4 * e;
        }
        const float4 s = sum_parts(src, stride, s1);
        if (!cursor_ok(a, after(cur, s.x))) return done(false);
        sq = store_grad4(dst, s);
    } else if (blockIdx.x < NRED) {
        // s3 = 4 s1 partials per unit: lane q of a quad sums partials q s1 .. q s1 + s1 - 1 in
        // split order (all of a lane's loads in flight at once), the quad adds its four sums in
        // order; 1,600 units (dW1 columns 1792..1799, then dW3) in 25 workgroups
        const int vu = (blockIdx.x - NRF) * 64 + (t >> 2), q = t & 3;
        const float *src;
        size_t stride;
        uint16_t *dst;
        if (vu < 2 * H) {
            const int n = vu >> 1, f = NT1 * 64 + 4 * (vu & 1);
            src = w.part1t + (size_t)n * 8 + (f - NT1 * 64), stride = (size_t)H * 8, dst = g + a.off_w1 + (size_t)n * K1 + f;
        } else {
            const int e = vu - 2 * H;
            src = w.part3 + 4 * e, stride = (size_t)NZ * H, dst = g + a.off_w3 + 4 * e;
        }
        const float4 s = sum_parts(src + (size_t)q * s1 * stride, stride, s1);
        if (!cursor_ok(a, after(cur, s.x))) return done(false);
        float4 o[3];
#pragma unroll
        for (int k = 0; k < 3; k++)
            o[k] = make_float4(__shfl_down(s.x, k + 1), __shfl_down(s.y, k + 1), __shfl_down(s.z, k + 1), __shfl_down(s.w, k + 1));
        if (q == 0) {
            const float4 tot = make_float4(((s.x + o[0].x) + o[1].x) + o[2].x, ((s.y + o[0].y) + o[1].y) + o[2].y,
                                           ((s.z + o[0].z) + o[1].z) + o[2].z, ((s.w + o[0].w) + o[1].w) + o[2].w);
            sq = store_grad4(dst, tot);
        }
    } else {   // biases: 8 columns per workgroup, 32 lanes per column over the row partials
        const int col = 8 * (blockIdx.x - NRED) + (t >> 5), part = t & 31, nrows = mb / R;
        float s = 0.f;
        if (col <= 2 * H + NZ)
            for (int r0 = part; r0 < nrows; r0 += 256) {   // eight loads in flight
                float x[8];
#pragma unroll
                for (int j = 0; j < 8; j++) x[j] = r0 + 32 * j < nrows ? w.bpart[(size_t)(r0 + 32 * j) * BP + col] : 0.f;
#pragma unroll
                for (int j = 0; j < 8; j++) s += x[j];
            }
        s = row16_sum(xor16_sum(s));   // the column's 32 lanes, fixed order
        if (!cursor_ok(a, after(cur, s))) return done(false);
        if (part == 0 && col < 2 * H + NZ) {
            const uint16_t hb = rb(s);
            uint16_t *dst = col < H ? g + a.off_b1 + col : col < 2 * H ? g + a.off_b2 + (col - H) : g + a.off_b3 + (col - 2 * H);
            *dst = hb;
            sq = bf(hb) * bf(hb);
        } else if (part == 0 && col == 2 * H + NZ) {
            // the loss column: 0 * (minibatch loss sum) is +-0 when the loss is finite, which
            // leaves the norm bit-identical, and NaN otherwise, so k_adam sees a non-finite
            // loss as a non-finite norm
            sq = 0.f * s;
        }
    }
    const float tot = block_sum(sq, red);
    if (t == 0) w.npart[blockIdx.x] = tot;
    done(true);
}

// ---------------------------------------------------------------- k_adam
// Refresh the packed slots of flat parameters i0..i0+3 (i0 - each weight offset is a
// multiple of 4, so the four share a weight row and one 8-byte run of the row-ordered copies).
__device__ __forceinline__ void pack_param4(const D1PPOStep &a, uint16_t *wpk, int64_t i0, const uint16_t (&h)[4]) {
    const uint2 v = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
    int64_t e;
    if ((e = i0 - a.off_w1) >= 0 && e < (int64_t)H * K1) {
        const int n = (int)e / K1, k = (int)e - n * K1;
        *(uint2 *)(wpk + pk_w1(n, k)) = v;
    } else if ((e = i0 - a.off_w2) >= 0 && e < H * H) {
        const int n = (int)e >> 8, k = (int)e & 255;
        *(uint2 *)(wpk + pk_w2(n, k)) = v;
#pragma unroll
        for (int q = 0; q < 4; q++) wpk[pk_w2t(n, k + q)] = h[q];
    } else if ((e = i0 - a.off_w3) >= 0 && e < NZ * H) {
        const int j = (int)e >> 8, k = (int)e & 255;
        *(uint2 *)(wpk + pk_w3(j, k)) = v;
#pragma unroll
        for (int q = 0; q < 4; q++) wpk[pk_w3t(j, k + q)] = h[q];
    }
}
// Refresh every packed slot of flat parameter i with its bf16 value h.
__device__ __forceinline__ void pack_param(const D1PPOStep &a, uint16_t *wpk, int64_t i, uint16_t h) {
    int64_t e;
    if ((e = i - a.off_w1) >= 0 && e < (int64_t)H * K1) {
        wpk[pk_w1((int)e / K1, (int)e % K1)] = h;
    } else if ((e = i - a.off_w2) >= 0 && e < H * H) {
        wpk[pk_w2((int)(e >> 8), (int)(e & 255))] = h;
        wpk[pk_w2t((int)(e >> 8), (int)(e & 255))] = h;
    } else if ((e = i - a.off_w3) >= 0 && e < NZ * H) {
        wpk[pk_w3((int)(e >> 8), (int)(e & 255))] = h;
        wpk[pk_w3t((int)(e >> 8), (int)(e & 255))] = h;
    }
}

// Global-norm clip + Adam (torch.optim.Adam, no weight decay) over the flat buffers. Every
// workgroup re-sums the norm partials; t = step[1] (set by k_reduce); workgroup 0 stores it
// back to step[0] and advances the minibatch cursor. A non-finite norm (non-finite
// gradients, or a non-finite loss folded in by k_reduce) leaves every parameter, moment and
// the step count as they are and counts the step in step[2]; while step[2] is not zero
// every later step is skipped the same way, so the weights stay those of the last step
// before the first non-finite loss.
__global__ __launch_bounds__(256) void k_adam(D1PPOStep a, Work w) {
    __shared__ float red[4];
    const int flag = load_cursor(a.cursor + 1);
    const uint16_t *g = (const uint16_t *)a.g;
    uint16_t *pb = (uint16_t *)a.pb;
    // this lane's four parameters (launched with one group per lane), loaded before the
    // norm reduction so that both latencies overlap
    const int64_t i0 = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
    const bool mine = i0 < a.nparams;
    const int64_t il = mine ? i0 : 0;
    const uint2 gv = *(const uint2 *)(g + il);
    float4 pv = *(const float4 *)(a.p + il), mv = *(const float4 *)(a.m + il), vv = *(const float4 *)(a.v + il);
    static_assert(NRED + NBIASB > 512 && NRED + NBIASB <= 768, "three norm partials per lane");
    const int j = threadIdx.x;   // blockDim.x == 256; the three loads are in flight together
    const float n0 = w.npart[j], n1 = w.npart[j + 256], n2 = j + 512 < NRED + NBIASB ? w.npart[j + 512] : 0.f;
    if (after(flag, n0) == 0) return;   // checked once the loads above are in flight
    const float acc = ((0.f + n0) + n1) + n2;
    const float norm = sqrtf(block_sum(acc, red));
    if (!(norm <= 3.4028235e38f) || a.step[2] != 0.f) {   // NaN fails the comparison
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            a.step[2] += 1.f;
            a.cursor[0] += 1;
        }
        return;
    }
    const float coef = fminf(a.max_grad_norm / (norm + 1e-6f), 1.f);
    const float tt = a.step[1];
    const float bc1 = 1.f - powf(a.beta1, tt), bc2 = 1.f - powf(a.beta2, tt);
    const float step_size = a.lr / bc1, bc2s = sqrtf(bc2);
    if (mine) {
        const float gs[4] = {bf((uint16_t)gv.x), bf((uint16_t)(gv.x >> 16)), bf((uint16_t)gv.y), bf((uint16_t)(gv.y >> 16))};
        float *pp = &pv.x, *mm = &mv.x, *vq = &vv.x;
        uint16_t h[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float gi = gs[e] * coef;
            mm[e] = a.beta1 * mm[e] + (1.f - a.beta1) * gi;
            vq[e] = a.beta2 * vq[e] + (1.f - a.beta2) * gi * gi;
            pp[e] = pp[e] - step_size * mm[e] / (sqrtf(vq[e]) / bc2s + a.eps);
        }
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
            const uint32_t w2 = cvt2(pp[e], pp[e + 1]);
            h[e] = (uint16_t)(w2 & 0xFFFFu);
            h[e + 1] = (uint16_t)(w2 >> 16);
        }
        *(float4 *)(a.p + i0) = pv;
        *(float4 *)(a.m + i0) = mv;
        *(float4 *)(a.v + i0) = vv;
        *(uint2 *)(pb + i0) = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
        pack_param4(a, w.wpk, i0, h);
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        a.step[0] = tt;
        a.cursor[0] += 1;
    }
}

// d1_ppo_prepare: zero the packed copies (their padding slots stay zero), then pack every
// weight from pb.
__global__ __launch_bounds__(256) void k_pack_zero(uint16_t *wpk) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < P_END; i += gridDim.x * blockDim.x) wpk[i] = 0;
}
__global__ __launch_bounds__(256) void k_pack(D1PPOStep a, uint16_t *wpk) {
    const uint16_t *pb = (const uint16_t *)a.pb;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.nparams; i += (int64_t)gridDim.x * blockDim.x)
        pack_param(a, wpk, i, pb[i]);
}

struct Layout {
    size_t wpk, h1f, h2f, dh2f, dh1f, dzf, xf, bpart, part1, part2, part3, part1t, npart, total;
};
constexpr size_t round256(size_t bytes) { return (bytes + 255) / 256 * 256; }
constexpr Layout layout(int mb) {
    Layout L{};
    size_t off = 0;
    L.wpk = off, off += round256((size_t)P_END * 2);
    L.h1f = off, off += round256((size_t)H * mb * 2);
    L.h2f = off, off += round256((size_t)H * mb * 2);
    L.dh2f = off, off += round256((size_t)H * mb * 2);
    L.dh1f = off, off += round256((size_t)H * mb * 2);
    L.dzf = off, off += round256((size_t)32 * mb * 2);
    L.xf = off, off += round256((size_t)XB * 32 * mb);
    L.bpart = off, off += round256((size_t)(mb / R) * BP * 4);
    L.part1 = off, off += round256((size_t)(mb / KW) * H * K1 * 4);
    L.part2 = off, off += round256((size_t)(mb / KW) * H * H * 4);
    L.part3 = off, off += round256((size_t)(mb / KW3) * NZ * H * 4);
    L.part1t = off, off += round256((size_t)(mb / KW3) * H * 8 * 4);
    L.npart = off, off += round256((size_t)(NRED + NBIASB) * 4);
    L.total = off;
    return L;
}

// Validates everything but the work buffer; `base`/`bytes` is the work buffer to carve.
static int check_args(const D1PPOStep *s, char *base, int64_t bytes, Work *w) {
    if (!s) return D1_E_ARG;
    const D1PPOStep &a = *s;
    if (a.mb <= 0 || a.mb % KW || a.n < a.mb || a.n >= ((int64_t)1 << 31) || a.nparams % 4) return D1_E_ARG;
    if (!a.obs || !a.perm || !a.cursor || !a.actions || !a.logp_old || !a.adv || !a.ret || !a.p || !a.pb || !a.g ||
        !a.m || !a.v || !a.step || !a.loss_parts || !base)
        return D1_E_ARG;
    if ((uintptr_t)a.obs % 8 || (uintptr_t)a.pb % 16 || (uintptr_t)a.g % 16 || (uintptr_t)base % 256 ||
        (uintptr_t)a.p % 16 || (uintptr_t)a.m % 16 || (uintptr_t)a.v % 16)
        return D1_E_ARG;
    const int64_t offs[6] = {a.off_w1, a.off_b1, a.off_w2, a.off_b2, a.off_w3, a.off_b3};
    const int64_t sizes[6] = {(int64_t)H * K1, H, (int64_t)H * H, H, (int64_t)NZ * H, NZ};
    for (int i = 0; i < 6; i++)
        if (offs[i] < 0 || offs[i] % 8 || offs[i] + sizes[i] > a.nparams) return D1_E_ARG;
    const Layout L = layout(a.mb);
    if (bytes < (int64_t)L.total) return D1_E_ARG;
    w->wpk = (uint16_t *)(base + L.wpk);
    w->h1f = (uint16_t *)(base + L.h1f);
    w->h2f = (uint16_t *)(base + L.h2f);
    w->dh2f = (uint16_t *)(base + L.dh2f);
    w->dh1f = (uint16_t *)(base + L.dh1f);
    w->dzf = (uint16_t *)(base + L.dzf);
    w->xf = (uint8_t *)(base + L.xf);
    w->bpart = (float *)(base + L.bpart);
    w->part1 = (float *)(base + L.part1);
    w->part2 = (float *)(base + L.part2);
    w->part3 = (float *)(base + L.part3);
    w->part1t = (float *)(base + L.part1t);
    w->npart = (float *)(base + L.npart);
    return 0;
}
static int check_args(const D1PPOStep *s, Work *w) {
    if (!s) return D1_E_ARG;
    return check_args(s, (char *)s->work, s->work_bytes, w);
}

static void launch_pack(const D1PPOStep &a, const Work &w, hipStream_t st) {
    hipLaunchKernelGGL(k_pack_zero, dim3(256), dim3(256), 0, st, w.wpk);
    hipLaunchKernelGGL(k_pack, dim3(512), dim3(256), 0, st, a, w.wpk);
}
static void launch_step(const D1PPOStep &a, const Work &w, hipStream_t st) {
    const int s1 = a.mb / KW;
    hipLaunchKernelGGL(k_rows, dim3(a.mb / R), dim3(512), 0, st, a, w);
    hipLaunchKernelGGL(k_wgrad, dim3(NT1 * s1 + 4 * s1 + a.mb / KW3), dim3(256), 0, st, a, w);
    hipLaunchKernelGGL(k_reduce, dim3(NRED + NBIASB), dim3(256), 0, st, a, w);
    const int64_t nadam = (a.nparams / 4 + 255) / 256;   // one group of four parameters per lane
    hipLaunchKernelGGL(k_adam, dim3((unsigned)nadam), dim3(256), 0, st, a, w);
}

// ---------------------------------------------------------------- library-owned work buffer
// d1_ppo_step_static's work buffer: one per GPU, reserved when the code object is loaded on
// that device (every process that loads this library holds it, whether or not it calls the
// PPO step) until the process ends, sized for the largest minibatch it accepts. In host code `scratch` names a host-side
// stand-in, never the device array: the device address comes from hipGetSymbolAddress, once
// per device, with that device current.
constexpr size_t SCRATCH_BYTES = layout(D1_PPO_STATIC_MAX_MB).total;
static __device__ __align__(256) char scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
static std::mutex scratch_lock;
static char *scratch_ptr[MAX_DEVICES];

// The device address of this device's `scratch`, or null with *err set.
static char *scratch_base(int *err) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        *err = D1_E_ARG;
        return nullptr;
    }
    std::lock_guard<std::mutex> hold(scratch_lock);
    if (!scratch_ptr[dev]) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            *err = e != hipSuccess ? (int)e : D1_E_ARG;
            return nullptr;
        }
        scratch_ptr[dev] = (char *)ptr;
    }
    return scratch_ptr[dev];
}

}  // namespace d1q

extern "C" int64_t d1_ppo_work_bytes(int mb) {
    if (mb <= 0 || mb % d1q::KW) return D1_E_ARG;
    return (int64_t)d1q::layout(mb).total;
}

extern "C" int d1_ppo_prepare(const D1PPOStep *s, void *stream) {
    using namespace d1q;
    Work w;
    if (int e = check_args(s, &w)) return e;
    launch_pack(*s, w, (hipStream_t)stream);
    return (int)hipGetLastError();
}

extern "C" int d1_ppo_step(const D1PPOStep *s, void *stream) {
    using namespace d1q;
    Work w;
    if (int e = check_args(s, &w)) return e;
    launch_step(*s, w, (hipStream_t)stream);
    return (int)hipGetLastError();
}

extern "C" int d1_ppo_step_static(const D1PPOStep *s, void *stream) {
    using namespace d1q;
    if (!s) return D1_E_ARG;
    if (s->mb > D1_PPO_STATIC_MAX_MB) return D1_E_SCRATCH;
    int err = 0;
    char *base = scratch_base(&err);
    if (!base) return err;
    Work w;
    if (int e = check_args(s, base, (int64_t)SCRATCH_BYTES, &w)) return e;
    const hipStream_t st = (hipStream_t)stream;
    launch_pack(*s, w, st);   // the packed weight copies are rebuilt from pb on every call
    launch_step(*s, w, st);
    return (int)hipGetLastError();
}
