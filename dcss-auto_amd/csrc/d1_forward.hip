// d1hip: the rollout policy forward as one MFMA kernel for MI355X (gfx950).
//
// logits, value = head(relu(relu(obs W1^T + b1) W2^T + b2)) for the BASELINE policy
// (gpu-d1/scripts/run_ring_ablations.py:209-223 with 1800 -> 256 -> 256 ReLU and a
// 16-logit + value head): obs uint8 [M, 1800] read directly (every byte value is exact in
// bf16), bf16 weights packed once per weight update (d1_policy_pack), fp32 accumulation,
// each layer's output rounded to bf16 where the bf16 torch path rounds it, fp32 logits
// [M, 16] and value [M] out. One launch replaces the widening pass, three library GEMMs
// and the dtype copy of the rollout forward.
//
// Every layer is computed transposed, D = W x act^T (A operand = weight rows, B operand =
// 32 samples), so that a lane's D registers hold one sample's hidden units. A 256-lane
// workgroup owns 256 samples; wave w computes samples 64w..64w+63 as 2 x 8 tiles of 32x32.
//   layer 1  29 chunks of 64 inputs. Each chunk's W1 fragments (32 KB) are copied once per
//            workgroup into double-buffered LDS (1 KB contiguous per load instruction);
//            the observation fragments come straight from global memory two chunks
//            ahead and are widened to bf16 in registers.
//   layer 2  h1 never leaves registers: in tile (a, b) lane (l%32, h = l/32) register r
//            holds hidden unit 32b + 8(r/4) + 4h + r%4 of sample 32a + l%32, and K step s
//            of layer 2 takes registers 8(s%2)..8(s%2)+7 of tile (a, s/2) as its B operand
//            slots j = 0..7. Slot j of half h in step s therefore stands for hidden unit
//            k(s, h, j) = 32(s/2) + 16(s%2) + 8(j/4) + 4h + j%4, and W2 is packed in that
//            order. W2 and the head weights (144 KB) are staged in LDS once per workgroup,
//            in three rounds by K step, the last one in flight during layer 2's first 12
//            steps.
//   head     the same for h2 against a 32-row head (rows 17..31 zero).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/d1hip.h"
#include "d1_frag.h"
#include "d1_sample.h"

namespace d1t {

using namespace d1f;

constexpr int K1 = 1800, H = 256, NA = 16, NZ = 17, BM = 256;
constexpr int C1 = 29;                       // layer-1 K chunks (28 of 64 + inputs 1792..1799)
constexpr int PW1 = 0;                       // W1: [29 chunks][8 row blocks][4 steps][64 lanes][8]
constexpr int PW2 = PW1 + 8 * C1 * 4 * 512;  // W2: [8 row blocks][16 steps][64][8], K order k(s, h, j)
constexpr int PW3 = PW2 + 8 * 16 * 512;      // head: [16 steps][64][8], rows 17..31 zero
constexpr int PEND = PW3 + 16 * 512;
constexpr int NSTAGE = (PEND - PW2) / 8;     // 16-byte pieces of W2 + head staged per workgroup (9216)
constexpr int LDS_W = NSTAGE * 16;           // 147,456 B (the layer-1 W1 buffers, 64 KB, alias its start)
constexpr int LDS_BYTES = LDS_W + 2 * 320 * 2;   // + biases b1 | b2 | head bias (padded to 32)
static_assert(2 * 2048 * 16 <= LDS_W, "W1 double buffer inside the staging area");
static_assert(NSTAGE % 256 == 0, "whole staging rounds");

// Autoregressive head (BASELINE C5, dcss-auto_amd/policy.py ARPolicy): the trunk head above
// holds the verb logits (rows 0-7, rows 8-15 zero) and the value (row 16); the target MLP's
// trunk part t1[:, :256] is two more 32-row head tiles, its verb-embedding part enters as the
// table ev[verb][64] = t1[:, 256:] . embedding[verb] (bf16, computed by torch once per weight
// update), and its output layer t2 (25 x 64) is one more MFMA tile over K = 64. The packed
// buffer continues after PEND: the two t1 tiles [2][16 steps][64][8] in the head's K order,
// t2 [4 steps][64][8] with hidden unit kperm(s, h, j), and ev [8][64].
constexpr int NV = 8, NT = 25, TH = 64;
constexpr int PA1 = PEND;                    // t1 trunk columns: 2 tiles x 16 steps
constexpr int PA2 = PA1 + 2 * 16 * 512;      // t2: 4 steps, rows 25..31 zero
constexpr int PAE = PA2 + 4 * 512;           // ev [8][64]
constexpr int PAEND = PAE + NV * TH;
constexpr int NSTAGE_AR = (PAEND - PA1) / 8; // 16-byte pieces restaged after layer 2 (2,368)
constexpr int LDS_BYTES_AR = LDS_BYTES + (TH + 32) * 2;   // + t1 bias (64) | t2 bias (padded to 32)
static_assert(NSTAGE_AR <= 8 * 16 * 64, "the AR pieces fit in the W2 area");

// hidden unit of B slot j, lane half h, layer-2/head K step s
__host__ __device__ constexpr int kperm(int s, int h, int j) {
    return 32 * (s >> 1) + 16 * (s & 1) + 8 * (j >> 2) + 4 * h + (j & 3);
}

// Outputs of the autoregressive epilogue (null pointers are skipped; action, logp and value
// are required)
struct ArOut {
    const uint16_t *bt;     // t1 bias [64] | t2 bias [25] (bf16)
    int32_t *verb, *target;
    float *verb_logits;     // [M, 8]
    float *target_logits;   // [M, 25]: the drawn verb's row
};

// a register-array element chosen at run time without a run-time register index (which
// would send the array to scratch): a select chain
template <int K>
__device__ __forceinline__ float sel(const float (&r)[K], int j) {
    float v = r[0];
#pragma unroll
    for (int q = 1; q < K; q++) v = j == q ? r[q] : v;
    return v;
}
__device__ __forceinline__ float bfr(float x) { return __uint_as_float(cvt2(x, 0.f) << 16); }   // bf16-rounded
__device__ __forceinline__ float bhalf(u32x2 w, int i) {
    return bf((uint16_t)((i < 2 ? w.x : w.y) >> (16 * (i & 1))));
}

// The autoregressive head after layer 2 (h2 in hf, B-fragment order). Head tiles: tile 0
// (verb logits rows 0-7, value row 16) staged with W2, the two t1 tiles at pieces [0, 2048).
// Lane half h draws for sample block h (sample m0 + 32h + lr): it gathers the block's eight
// verb logits from its partner lane (l ^ 32), draws the verb with u0, and the partner learns
// it back; each lane then forms z = tanh(bf16(ht + ev[verb])) for its 32 hidden units of both
// blocks in the B-fragment order of the t2 tile (unit kperm(s, h, j) in step s, slot j), and
// one K = 64 MFMA chain gives the drawn verb's 25 target logits, which the lane halves gather
// as they did the verb logits and draw with u1. Rounding follows the bf16 torch forward:
// every linear output is rounded once after its bias, ht + ev and tanh are rounded to bf16.
__device__ __forceinline__ void ar_epilogue(const u32x4 *stage, const uint16_t *bl, const bf16x8 (&hf)[2][16],
                                            int lane, int lr, int lh, int m0, int M, uint32_t key0, uint32_t key1,
                                            uint32_t tstep, float *__restrict__ value, int64_t *__restrict__ actions,
                                            float *__restrict__ logp, const ArOut &ar) {
    floatx16 z0[2] = {}, z1[2] = {}, z2[2] = {};
    {
        const u32x4 *w0p = stage + 8 * 16 * 64 + lane, *w1p = stage + lane, *w2p = stage + 16 * 64 + lane;
#pragma unroll
        for (int s = 0; s < 16; s++) {
            const bf16x8 f0 = as_bf(w0p[s * 64]), f1 = as_bf(w1p[s * 64]), f2 = as_bf(w2p[s * 64]);
#pragma unroll
            for (int a = 0; a < 2; a++) {
                z0[a] = mfma(f0, hf[a][s], z0[a]);
                z1[a] = mfma(f1, hf[a][s], z1[a]);
                z2[a] = mfma(f2, hf[a][s], z2[a]);
            }
        }
    }
    const uint16_t *b3l = bl + 512, *btl = bl + 544;
    const uint32_t hm = 0u - (uint32_t)lh;
    auto pick = [&](float if0, float if1) {
        return __uint_as_float((__float_as_uint(if1) & hm) | (__float_as_uint(if0) & ~hm));
    };
    // verb logits 4lh..4lh+3 of block a in z0[a][0..3], the value (lane half 0) in z0[a][8]
    float ov[2][4], val[2];
    {
        const u32x2 bw = *(const u32x2 *)(b3l + 4 * lh);
#pragma unroll
        for (int a = 0; a < 2; a++) {
#pragma unroll
            for (int i = 0; i < 4; i++) ov[a][i] = bfr(z0[a][i] + bhalf(bw, i));
            val[a] = bfr(z0[a][8] + bf(b3l[16]));
        }
    }
    float l8[NV];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float q = __shfl_xor(pick(ov[1][i], ov[0][i]), 32);
        l8[i] = pick(ov[0][i], q);
        l8[4 + i] = pick(q, ov[1][i]);
    }
    const int m = m0 + 32 * lh + lr;
    uint32_t w0, w1;
    d1s::philox_w01(0u, tstep, (uint32_t)m, 3u, key0, key1, w0, w1);
    int v;
    float lv;
    d1s::cat_core([&](int j) { return l8[j]; }, NV, d1s::unit24(w0), v, lv);
    const int vq = __shfl_xor(v, 32);
    const int va[2] = {lh ? vq : v, lh ? v : vq};   // the drawn verbs of blocks 0 and 1 of sample row lr

    // t2's B operand: z of this lane's hidden units for both blocks
    bf16x8 hz[2][4];
    const uint16_t *evl = (const uint16_t *)(stage + (PAE - PA1) / 8);
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int T = 0; T < 2; T++)
#pragma unroll
            for (int g = 0; g < 4; g++) {   // registers 4g..4g+3: units 32T + 8g + 4lh + 0..3
                const int u0 = 32 * T + 8 * g + 4 * lh;
                const u32x2 bw = *(const u32x2 *)(btl + u0);
                const u32x2 ew = *(const u32x2 *)(evl + va[a] * TH + u0);
                float zz[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float ht = bfr((T ? z2[a] : z1[a])[4 * g + i] + bhalf(bw, i));
                    zz[i] = tanhf(bfr(ht + bhalf(ew, i)));
                }
                u32x4 w = __builtin_bit_cast(u32x4, hz[a][2 * T + (g >> 1)]);
                w[2 * (g & 1)] = cvt2(zz[0], zz[1]);
                w[2 * (g & 1) + 1] = cvt2(zz[2], zz[3]);
                hz[a][2 * T + (g >> 1)] = as_bf(w);
            }
    floatx16 zt[2] = {};
    {
        const u32x4 *w3p = stage + 2 * 16 * 64 + lane;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const bf16x8 f = as_bf(w3p[s * 64]);
#pragma unroll
            for (int a = 0; a < 2; a++) zt[a] = mfma(f, hz[a][s], zt[a]);
        }
    }
    // target row 8g + 4lh + i of block a sits in register 4g + i; lane half h gathers block h's
    float tl[NT];
    {
        const uint16_t *bt2 = btl + TH;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const u32x2 bw = *(const u32x2 *)(bt2 + 8 * g + 4 * lh);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float o0 = bfr(zt[0][4 * g + i] + bhalf(bw, i)), o1 = bfr(zt[1][4 * g + i] + bhalf(bw, i));
                const float q = __shfl_xor(pick(o1, o0), 32);
                if (8 * g + i < NT) tl[8 * g + i] = pick(o0, q);
                if (8 * g + 4 + i < NT) tl[8 * g + 4 + i] = pick(q, o1);
            }
        }
    }
    int tg;
    float lt;
    d1s::cat_core([&](int j) { return tl[j]; }, NT, d1s::unit24(w1), tg, lt);
    if (m < M) {
        actions[m] = d1s::ar_action(v, tg);
        logp[m] = lv + lt;
        if (ar.verb) ar.verb[m] = v;
        if (ar.target) ar.target[m] = tg;
        if (ar.verb_logits) {
            *(float4 *)(ar.verb_logits + (size_t)m * NV) = make_float4(l8[0], l8[1], l8[2], l8[3]);
            *(float4 *)(ar.verb_logits + (size_t)m * NV + 4) = make_float4(l8[4], l8[5], l8[6], l8[7]);
        }
        if (ar.target_logits) {
#pragma unroll
            for (int j = 0; j < NT; j++) ar.target_logits[(size_t)m * NT + j] = tl[j];
        }
    }
#pragma unroll
    for (int a = 0; a < 2; a++) {
        const int ma = m0 + 32 * a + lr;
        if (ma < M && lh == 0) value[ma] = val[a];
    }
}

// MODE 0: logits and value. MODE 1: the epilogue also draws each sample's action with the
// counter-RNG sampler (d1_sample.h, the arithmetic of d1_sample) at step t = (t_dev ? *t_dev :
// 0) + t_add; logits may then be null. MODE 2: the autoregressive head with its two-stage
// sample (the arithmetic of d1_sample_ar).
template <int MODE>
__global__ __launch_bounds__(256) void k_policy(const uint8_t *__restrict__ obs, int M, const uint16_t *__restrict__ wpk,
                                                const uint16_t *__restrict__ b1, const uint16_t *__restrict__ b2,
                                                const uint16_t *__restrict__ b3, float *__restrict__ logits,
                                                float *__restrict__ value, uint32_t key0, uint32_t key1,
                                                const uint32_t *__restrict__ t_dev, uint32_t t_add,
                                                int64_t *__restrict__ actions, float *__restrict__ logp, ArOut ar) {
    constexpr bool SAMPLE = MODE == 1, AR = MODE == 2;
    __shared__ __align__(16) uint8_t lds[AR ? LDS_BYTES_AR : LDS_BYTES];
    const int t = threadIdx.x, lane = t & 63, lr = lane & 31, lh = lane >> 5;
    u32x4 *stage = (u32x4 *)lds;                           // W1 double buffer, later W2 + head
    uint16_t *bl = (uint16_t *)(lds + LDS_W);              // [0,256) b1, [256,512) b2 (both permuted, below), [512,544) head bias
    const int m0 = blockIdx.x * BM + 64 * (t >> 6);
    // the sampler's step, read now: loaded where it is used, at the end, its latency was
    // the last thing every workgroup waited for (the AR build keeps the late load, which
    // costs it no registers through the trunk)
    const uint32_t tstep = SAMPLE ? (t_dev ? *t_dev : 0u) + t_add : 0u;

    {   // b1 and b2 in conversion order: unit 32b + 8g + 4h + i at 32b + 16h + 4g + i
        const int u = t, pu = (u & ~31) + 16 * ((u >> 2) & 1) + 4 * ((u >> 3) & 3) + (u & 3);
        bl[pu] = b1[u];
        bl[256 + pu] = b2[u];
    }
    if (t < 32) bl[512 + t] = t < NZ ? b3[t] : 0;
    if (AR && t < TH + 32) bl[544 + t] = t < TH + NT ? ar.bt[t] : 0;

    floatx16 acc[2][8];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 8; b++) acc[a][b] = floatx16{};

    // ---- layer 1. W1 chunk c (32 KB, contiguous in the packed buffer) is loaded two chunks
    // ahead into register slot c % 2 (8 pieces of 16 bytes per lane) and stored into LDS
    // buffer c % 2 one chunk ahead. Observation fragments (sample 32a + lr, bytes
    // 64ch + 32lh + 8q .. +7) are loaded two chunks ahead into three named register slots
    // (chunk c in slot c % 3). No load sits behind a branch: samples at or past M read row
    // M-1 (their outputs are not stored) and the chunk-28 addresses past input 1799 are
    // clamped to 1792, where the packed W1 is zero.
    const uint8_t *arow[2];
#pragma unroll
    for (int a = 0; a < 2; a++) arow[a] = obs + (size_t)min(m0 + 32 * a + lr, M - 1) * K1;
    u32x2 vA0[2][4], vA1[2][4], vA2[2][4];
    u32x4 vb0[8], vb1[8];
    auto aload = [&](u32x2 (&va)[2][4], int ch) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int k = min(64 * ch + 32 * lh + 8 * q, K1 - 8);
#pragma unroll
            for (int a = 0; a < 2; a++) va[a][q] = *(const u32x2 *)(arow[a] + k);
        }
    };
    // pieces t + 256i of chunk ch (row block p >> 8, step (p >> 6) & 3, lane p & 63), stored
    // at the same piece index of an LDS buffer
    auto bload = [&](u32x4 (&vb)[8], int ch) {
        const u32x4 *src = (const u32x4 *)(wpk + PW1) + (size_t)ch * 2048 + t;
#pragma unroll
        for (int i = 0; i < 8; i++) vb[i] = src[256 * i];
    };
    auto bstore = [&](const u32x4 (&vb)[8], int buf) {
#pragma unroll
        for (int i = 0; i < 8; i++) stage[buf * 2048 + t + 256 * i] = vb[i];
    };
    // the next step's 8 W1 fragments are read from LDS while this step's 16 MFMAs run
    auto mma1 = [&](int buf, const bf16x8 (&fa)[2][4]) {
        const u32x4 *src = stage + buf * 2048 + lane;
        bf16x8 fw[8], fn[8];
#pragma unroll
        for (int b = 0; b < 8; b++) fw[b] = as_bf(src[b * 4 * 64]);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (q < 3) {
#pragma unroll
                for (int b = 0; b < 8; b++) fn[b] = as_bf(src[(b * 4 + q + 1) * 64]);
            }
#pragma unroll
            for (int b = 0; b < 8; b++)
#pragma unroll
                for (int a = 0; a < 2; a++) acc[a][b] = mfma(fw[b], fa[a][q], acc[a][b]);
            if (q < 3) {
#pragma unroll
                for (int b = 0; b < 8; b++) fw[b] = fn[b];
            }
        }
    };
    // The empty asm makes the slot's value opaque where it is consumed: without it the
    // compiler computes the widening right behind the load, two chunks early, and waits
    // for the observation bytes there, which undoes the prefetch.
    auto widen_slot = [&](u32x2 (&v)[2][4], bf16x8 (&fa)[2][4]) {
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                asm volatile("" : "+v"(v[a][q]));
                fa[a][q] = widen8(v[a][q].x, v[a][q].y);
            }
    };
    // chunk ch < 28: issue chunk ch + 2's W1 and observation loads (the W1 loads first),
    // multiply chunk ch, store chunk ch + 1's W1 pieces (loaded a step earlier: loads retire
    // in issue order, so this waits for them and not for this step's loads) into the other
    // buffer, meet at the barrier. The scheduling groups pin the order: the first step's 8
    // fragment reads, then 2 MFMAs per LDS fragment read with one global load after each
    // of the first 12 pairs, and the LDS stores one per MFMA pair over the last 16 MFMAs:
    // issued in one block (loads first, stores last), they left the MFMA pipe idle while
    // they issued (layer 1: 97.7K -> 77.8K cycles per workgroup).
    auto step = [&](int ch, u32x2 (&vcur)[2][4], u32x2 (&vnext)[2][4], u32x4 (&vbl)[8], const u32x4 (&vbs)[8],
                    bool more) {
        bf16x8 fa[2][4];
        widen_slot(vcur, fa);
        if (more) bload(vbl, ch + 2);
        aload(vnext, ch + 2);
        mma1(ch & 1, fa);
        bstore(vbs, (ch + 1) & 1);
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
        if (more) {
#pragma unroll
            for (int i = 0; i < 12; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
#pragma unroll
            for (int i = 4; i < 12; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
        }
#pragma unroll
        for (int i = 12; i < 24; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
        }
        __syncthreads();
    };
    bload(vb0, 0);
    aload(vA0, 0);
    bload(vb1, 1);
    aload(vA1, 1);
    bstore(vb0, 0);
    __syncthreads();
    for (int ch = 0; ch < 24; ch += 6) {   // chunk c: observation slot c % 3, W1 slot c % 2
        step(ch, vA0, vA2, vb0, vb1, true);
        step(ch + 1, vA1, vA0, vb1, vb0, true);
        step(ch + 2, vA2, vA1, vb0, vb1, true);
        step(ch + 3, vA0, vA2, vb1, vb0, true);
        step(ch + 4, vA1, vA0, vb0, vb1, true);
        step(ch + 5, vA2, vA1, vb1, vb0, true);
    }
    step(24, vA0, vA2, vb0, vb1, true);
    step(25, vA1, vA0, vb1, vb0, true);
    step(26, vA2, vA1, vb0, vb1, true);
    step(27, vA0, vA2, vb1, vb0, false);   // stores chunk 28's W1 pieces in buffer 0
    {                                       // chunk 28 (inputs 1792..1799) sits in slot 1
        bf16x8 fa[2][4];
        widen_slot(vA1, fa);
        mma1(0, fa);
    }
    __syncthreads();   // every wave is done with the W1 buffers before they are overwritten

    // bias + ReLU + bf16 rounding (hardware pack) of acc into B fragments: fragment s of sample block a takes
    // registers 8(s%2)..+7 of tile (a, s/2); register 4g + i is hidden unit 32b + 8g + 4lh + i
    bf16x8 hf[2][16];
    // (bias: this layer's 256 values in conversion order, the 16 of block b and lane half h
    // contiguous at 32b + 16h)
    auto to_frags = [&](const uint16_t *bias) {
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const u32x4 r0 = *(const u32x4 *)(bias + 32 * b + 16 * lh), r1 = *(const u32x4 *)(bias + 32 * b + 16 * lh + 8);
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const uint32_t bx = g == 0 ? r0.x : g == 1 ? r0.z : g == 2 ? r1.x : r1.z;
                const uint32_t by = g == 0 ? r0.y : g == 1 ? r0.w : g == 2 ? r1.y : r1.w;
                const float bb[4] = {bf(bx & 0xFFFFu), bf(bx >> 16), bf(by & 0xFFFFu), bf(by >> 16)};
#pragma unroll
                for (int a = 0; a < 2; a++) {
                    const int s = 2 * b + (g >> 1), j0 = 4 * (g & 1);
                    u32x4 w = __builtin_bit_cast(u32x4, hf[a][s]);
                    w[j0 / 2] = cvt2(fmaxf(acc[a][b][4 * g] + bb[0], 0.f), fmaxf(acc[a][b][4 * g + 1] + bb[1], 0.f));
                    w[j0 / 2 + 1] = cvt2(fmaxf(acc[a][b][4 * g + 2] + bb[2], 0.f), fmaxf(acc[a][b][4 * g + 3] + bb[3], 0.f));
                    hf[a][s] = as_bf(w);
                }
            }
        }
    };
    // stage W2 + head into LDS in 3 rounds of 12 pieces per lane, by K step: round 0 holds
    // W2's steps 0..5, round 1 steps 6..11, round 2 steps 12..15 and the head. Rounds 0 and 1
    // are in flight during the h1 conversion; round 2 is in flight during layer 2's first 12
    // steps and is stored after them.
    constexpr int RND = NSTAGE / 256 / 3;
    static_assert(RND == 12 && NSTAGE == 8 * 16 * 64 + 16 * 64, "three rounds of 3,072 pieces");
    auto spiece = [&](int r, int i) {   // piece of round r, item i (the same index in wpk and in LDS)
        const int q = t + 256 * i;
        if (r == 2 && q >= 2048) return 8 * 16 * 64 + (q - 2048);   // the head
        return ((q >> 6 & 7) * 16 + 6 * r + (q >> 9)) * 64 + (q & 63);
    };
    u32x4 sv[RND], sv1[RND];
#pragma unroll
    for (int i = 0; i < RND; i++) sv[i] = *(const u32x4 *)(wpk + PW2 + (size_t)spiece(0, i) * 8);
#pragma unroll
    for (int i = 0; i < RND; i++) sv1[i] = *(const u32x4 *)(wpk + PW2 + (size_t)spiece(1, i) * 8);
    to_frags(bl);
#pragma unroll
    for (int i = 0; i < RND; i++) stage[spiece(0, i)] = sv[i];
#pragma unroll
    for (int i = 0; i < RND; i++) stage[spiece(1, i)] = sv1[i];
#pragma unroll
    for (int i = 0; i < RND; i++) sv[i] = *(const u32x4 *)(wpk + PW2 + (size_t)spiece(2, i) * 8);
    __syncthreads();   // rounds 0 and 1 visible

    // ---- layer 2
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 8; b++) acc[a][b] = floatx16{};
    {
        const u32x4 *w2 = stage + lane;
        auto l2step = [&](int s) {
            bf16x8 fw[8];
#pragma unroll
            for (int b = 0; b < 8; b++) fw[b] = as_bf(w2[(b * 16 + s) * 64]);
#pragma unroll
            for (int b = 0; b < 8; b++)
#pragma unroll
                for (int a = 0; a < 2; a++) acc[a][b] = mfma(fw[b], hf[a][s], acc[a][b]);
        };
#pragma unroll
        for (int s = 0; s < 12; s++) l2step(s);
#pragma unroll
        for (int i = 0; i < RND; i++) stage[spiece(2, i)] = sv[i];
        __syncthreads();   // round 2 visible
#pragma unroll
        for (int s = 12; s < 16; s++) l2step(s);
    }
    if constexpr (AR) {
        // The AR pieces go where W2 was: their loads are in flight while h2 is converted,
        // and the LDS stores wait until every wave has read its last W2 fragment.
        constexpr int RA = (NSTAGE_AR + 255) / 256;
        u32x4 va[RA];
#pragma unroll
        for (int i = 0; i < RA; i++) {
            const int piece = min(t + 256 * i, NSTAGE_AR - 1);
            va[i] = *(const u32x4 *)(wpk + PA1 + (size_t)piece * 8);
        }
        to_frags(bl + 256);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < RA; i++)
            if (t + 256 * i < NSTAGE_AR) stage[t + 256 * i] = va[i];
        __syncthreads();
    } else {
        to_frags(bl + 256);
    }

    if constexpr (AR) {
        ar_epilogue(stage, bl, hf, lane, lr, lh, m0, M, key0, key1, (t_dev ? *t_dev : 0u) + t_add, value, actions,
                    logp, ar);
        return;
    }
    // ---- head: z[a] lane (lr, lh) register r = output 8(r/4) + 4lh + r%4 of sample 32a + lr
    floatx16 z[2] = {};
    {
        const u32x4 *w3 = stage + 8 * 16 * 64 + lane;
        bf16x8 fw[16];   // all 16 head fragments read first: one LDS wait instead of sixteen
#pragma unroll
        for (int s = 0; s < 16; s++) fw[s] = as_bf(w3[s * 64]);
#pragma unroll
        for (int s = 0; s < 16; s++)
#pragma unroll
            for (int a = 0; a < 2; a++) z[a] = mfma(fw[s], hf[a][s], z[a]);
    }
    const uint16_t *b3l = bl + 512;
    // the head output is bf16 (rounded once after the bias), widened to fp32; for sample block
    // a this lane holds logits 4lh..4lh+3 (o[a][0..3]) and 8+4lh..8+4lh+3 (o[a][4..7]), lane
    // half 0 the value
    float o[2][8], v[2];
#pragma unroll
    for (int a = 0; a < 2; a++) {
#pragma unroll
        for (int g = 0; g < 2; g++)
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                const uint32_t w = cvt2(z[a][4 * g + i] + bf(b3l[8 * g + 4 * lh + i]),
                                        z[a][4 * g + i + 1] + bf(b3l[8 * g + 4 * lh + i + 1]));
                o[a][4 * g + i] = __uint_as_float(w << 16);
                o[a][4 * g + i + 1] = __uint_as_float(w & 0xFFFF0000u);
            }
        v[a] = __uint_as_float(cvt2(z[a][8] + bf(b3l[16]), 0.f) << 16);
    }
    if (SAMPLE) {
        // lane half h samples block a = h: it keeps its own half of that block's row and
        // receives the other half from its partner lane (l ^ 32), which sends the half of
        // the partner's own block that this lane lacks
        // value blends by mask (a ternary between array elements is turned into a run-time
        // index into a stack copy of the array)
        const uint32_t hm = 0u - (uint32_t)lh;
        auto pick = [&](float if0, float if1) {
            return __uint_as_float((__float_as_uint(if1) & hm) | (__float_as_uint(if0) & ~hm));
        };
        float p[8], l16[16];
#pragma unroll
        for (int j = 0; j < 8; j++) p[j] = __shfl_xor(pick(o[1][j], o[0][j]), 32);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            l16[i] = pick(o[0][i], p[i]);
            l16[4 + i] = pick(p[i], o[1][i]);
            l16[8 + i] = pick(o[0][4 + i], p[4 + i]);
            l16[12 + i] = pick(p[4 + i], o[1][4 + i]);
        }
        const int m = m0 + 32 * lh + lr;
        if (m < M) {
            auto lg = [&](int j) {   // a select chain: no register array indexed at run time
                float r = l16[0];
#pragma unroll
                for (int q = 1; q < 16; q++) r = j == q ? l16[q] : r;
                return r;
            };
            int act;
            float lp;
            d1s::sample_core(lg, NA, key0, key1, tstep, (uint32_t)m, act, lp);
            actions[m] = act;
            logp[m] = lp;
        }
    }
#pragma unroll
    for (int a = 0; a < 2; a++) {
        const int m = m0 + 32 * a + lr;
        if (m < M) {
            if (!SAMPLE || logits) {
#pragma unroll
                for (int g = 0; g < 2; g++)
                    *(float4 *)(logits + (size_t)m * NA + 8 * g + 4 * lh) =
                        make_float4(o[a][4 * g], o[a][4 * g + 1], o[a][4 * g + 2], o[a][4 * g + 3]);
            }
            if (lh == 0) value[m] = v[a];
        }
    }
}

// Packed weights, one thread per element (gather form: every element is written, padding
// as zero). Element e of a region: j = e & 7, lane = (e >> 3) & 63 (row lane % 32, half
// lane / 32), step = e >> 9 within the region's block/chunk index.
__global__ __launch_bounds__(256) void k_policy_pack(const uint16_t *__restrict__ w1, const uint16_t *__restrict__ w2,
                                                     const uint16_t *__restrict__ w3, uint16_t *__restrict__ wpk) {
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < PEND; e += gridDim.x * blockDim.x) {
        const int j = e & 7, ln = (e >> 3) & 63, r = ln & 31, h = ln >> 5;
        uint16_t v = 0;
        if (e < PW2) {   // W1 [chunk][block][q]: row 32 block + r, input 64 chunk + 32h + 8q + j
            const int q = (e >> 9) & 3, blk = (e >> 11) & 7, ch = e >> 14;
            const int k = 64 * ch + 32 * h + 8 * q + j;
            if (k < K1) v = w1[(size_t)(32 * blk + r) * K1 + k];
        } else if (e < PW3) {   // W2 [block][s]: row 32 block + r, hidden unit kperm(s, h, j)
            const int f = e - PW2, s = (f >> 9) & 15, blk = f >> 13;
            v = w2[(32 * blk + r) * H + kperm(s, h, j)];
        } else {   // head [s]: output r (< 17), hidden unit kperm(s, h, j)
            const int s = (e - PW3) >> 9;
            if (r < NZ) v = w3[r * H + kperm(s, h, j)];
        }
        wpk[e] = v;
    }
}

// The autoregressive head's part of the packed buffer, [PA1, PAEND), same element rule:
// the two t1 tiles (row 32T + r of t1, h2 unit kperm(s, h, j)), t2 (row r < 25, t1 unit
// kperm(s, h, j) for s < 4, i.e. all 64), then ev copied as [8][64].
__global__ __launch_bounds__(256) void k_policy_pack_ar(const uint16_t *__restrict__ t1w,
                                                        const uint16_t *__restrict__ t2w,
                                                        const uint16_t *__restrict__ ev, uint16_t *__restrict__ wpk) {
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < PAEND - PA1; e += gridDim.x * blockDim.x) {
        const int j = e & 7, ln = (e >> 3) & 63, r = ln & 31, h = ln >> 5;
        uint16_t v = 0;
        if (e < PA2 - PA1) {
            const int s = (e >> 9) & 15, tile = e >> 13;
            v = t1w[(32 * tile + r) * (H + 16) + kperm(s, h, j)];
        } else if (e < PAE - PA1) {
            const int s = (e - (PA2 - PA1)) >> 9;
            if (r < NT) v = t2w[r * TH + kperm(s, h, j)];
        } else {
            v = ev[e - (PAE - PA1)];
        }
        wpk[PA1 + e] = v;
    }
}

}  // namespace d1t

extern "C" int64_t d1_policy_packed_elems(void) { return d1t::PEND; }
extern "C" int64_t d1_policy_ar_packed_elems(void) { return d1t::PAEND; }

extern "C" int d1_policy_ar_pack(const void *w1, const void *w2, const void *w3, const void *t1w, const void *t2w,
                                 const void *ev, void *wpk, void *stream) {
    if (!w1 || !w2 || !w3 || !t1w || !t2w || !ev || !wpk || (uintptr_t)wpk % 16) return D1_E_ARG;
    hipLaunchKernelGGL(d1t::k_policy_pack, dim3((d1t::PEND + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t *)w1, (const uint16_t *)w2, (const uint16_t *)w3, (uint16_t *)wpk);
    hipLaunchKernelGGL(d1t::k_policy_pack_ar, dim3((d1t::PAEND - d1t::PA1 + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, (const uint16_t *)t1w, (const uint16_t *)t2w, (const uint16_t *)ev,
                       (uint16_t *)wpk);
    return (int)hipGetLastError();
}

extern "C" int d1_policy_fwd_sample_ar(const uint8_t *obs, int M, const void *wpk, const void *b1, const void *b2,
                                       const void *b3, const void *bt, uint64_t seed, const uint32_t *t_dev,
                                       uint32_t t_add, float *value, int64_t *action, float *logp, int32_t *verb,
                                       int32_t *target, float *verb_logits, float *target_logits, void *stream) {
    if (M < 0 || (M > 0 && (!obs || !wpk || !b1 || !b2 || !b3 || !bt || !value || !action || !logp))) return D1_E_ARG;
    if ((uintptr_t)obs % 8 || (uintptr_t)wpk % 16 || (uintptr_t)bt % 8 || (uintptr_t)verb_logits % 16)
        return D1_E_ARG;
    if (M == 0) return 0;
    const d1t::ArOut ar{(const uint16_t *)bt, verb, target, verb_logits, target_logits};
    hipLaunchKernelGGL(d1t::k_policy<2>, dim3((M + d1t::BM - 1) / d1t::BM), dim3(256), 0, (hipStream_t)stream, obs, M,
                       (const uint16_t *)wpk, (const uint16_t *)b1, (const uint16_t *)b2, (const uint16_t *)b3, nullptr,
                       value, (uint32_t)seed, (uint32_t)(seed >> 32), t_dev, t_add, action, logp, ar);
    return (int)hipGetLastError();
}

extern "C" int d1_policy_pack(const void *w1, const void *w2, const void *w3, void *wpk, void *stream) {
    if (!w1 || !w2 || !w3 || !wpk || (uintptr_t)wpk % 16) return D1_E_ARG;
    hipLaunchKernelGGL(d1t::k_policy_pack, dim3((d1t::PEND + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t *)w1, (const uint16_t *)w2, (const uint16_t *)w3, (uint16_t *)wpk);
    return (int)hipGetLastError();
}

extern "C" int d1_policy_fwd(const uint8_t *obs, int M, const void *wpk, const void *b1, const void *b2, const void *b3,
                             float *logits, float *value, void *stream) {
    if (M < 0 || (M > 0 && (!obs || !wpk || !b1 || !b2 || !b3 || !logits || !value))) return D1_E_ARG;
    if ((uintptr_t)obs % 8 || (uintptr_t)wpk % 16 || (uintptr_t)logits % 16) return D1_E_ARG;
    if (M == 0) return 0;
    hipLaunchKernelGGL(d1t::k_policy<0>, dim3((M + d1t::BM - 1) / d1t::BM), dim3(256), 0, (hipStream_t)stream, obs,
                       M, (const uint16_t *)wpk, (const uint16_t *)b1, (const uint16_t *)b2, (const uint16_t *)b3, logits,
                       value, 0u, 0u, nullptr, 0u, nullptr, nullptr, d1t::ArOut{});
    return (int)hipGetLastError();
}

extern "C" int d1_policy_fwd_sample(const uint8_t *obs, int M, const void *wpk, const void *b1, const void *b2,
                                    const void *b3, uint64_t seed, const uint32_t *t_dev, uint32_t t_add, float *logits,
                                    float *value, int64_t *actions, float *logp, void *stream) {
    if (M < 0 || (M > 0 && (!obs || !wpk || !b1 || !b2 || !b3 || !value || !actions || !logp))) return D1_E_ARG;
    if ((uintptr_t)obs % 8 || (uintptr_t)wpk % 16 || (uintptr_t)logits % 16) return D1_E_ARG;
    if (M == 0) return 0;
    hipLaunchKernelGGL(d1t::k_policy<1>, dim3((M + d1t::BM - 1) / d1t::BM), dim3(256), 0, (hipStream_t)stream, obs,
                       M, (const uint16_t *)wpk, (const uint16_t *)b1, (const uint16_t *)b2, (const uint16_t *)b3, logits,
                       value, (uint32_t)seed, (uint32_t)(seed >> 32), t_dev, t_add, actions, logp, d1t::ArOut{});
    return (int)hipGetLastError();
}
