// d1hip: the policy trunk's first layer as one MFMA kernel for MI355X (gfx950).
//
// h1 = relu(obs @ W1^T + b1) with obs uint8 [M, 1800] read directly (every byte value
// is exact in bf16), W1 bf16 [256, 1800] (the torch Linear layout), b1 bf16 [256],
// fp32 accumulation, h1 bf16 [M, 256] rounded to nearest even. This replaces the
// separate uint8->bf16 widening pass and the library GEMM of the rollout forward
// (gpu-d1/scripts/run_ring_ablations.py:209-223 with the BASELINE 1800->256 layer).
//
// Tiling: a 256-lane workgroup owns 256 rows x all 256 columns; wave w computes rows
// 64w..64w+63 as 2x8 tiles of v_mfma_f32_32x32x16_bf16 (256 fp32 accumulators per
// lane; the 32x32 form sustains ~1.8 PFLOP/s at one wave per SIMD on this part).
// Operand lane layouts (checked on the hardware): A lane l holds A[l%32][8*(l/32) + j],
// B lane l holds B[8*(l/32) + j][l%32], D lane l holds D[8*(r/4) + 4*(l/32) + r%4][l%32]. A fragments (8 contiguous observation bytes) come straight
// from global memory; each 64-wide K slice of W1 is loaded once per workgroup into a
// double-buffered LDS tile (row n padded to 144 B) that the four waves share. K = 1800
// is walked in 29 steps of 64, the chunks at k >= 1800 read as zero; the next step's
// global loads are issued before the current step's 128 MFMAs.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/d1hip.h"

namespace d1t {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16;

constexpr int K1 = 1800, N1 = 256, BM = 256, KS = 64, KSTEPS = (K1 + KS - 1) / KS, BROW = 9;   // BROW: uint4 per LDS row of B (8 + 1 pad)

// two bytes of x (at bit 8s) -> two bf16 in one dword (exact: byte values need 8 bits)
__device__ __forceinline__ uint32_t widen2(uint32_t x, int s) {
    uint32_t lo = __float_as_uint((float)((x >> (8 * s)) & 255u)) >> 16;
    uint32_t hi = __float_as_uint((float)((x >> (8 * s + 8)) & 255u)) & 0xFFFF0000u;
    return lo | hi;
}
__device__ __forceinline__ bf16x8 widen8(uint2 v) {
    uint4 u = make_uint4(widen2(v.x, 0), widen2(v.x, 2), widen2(v.y, 0), widen2(v.y, 2));
    return __builtin_bit_cast(bf16x8, u);
}
__device__ __forceinline__ uint16_t f_to_bf16(float f) {   // round to nearest even (finite inputs)
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__global__ __launch_bounds__(256) void k_trunk1(const uint8_t *__restrict__ obs, int M,
                                                const uint16_t *__restrict__ w1, const uint16_t *__restrict__ b1,
                                                uint16_t *__restrict__ h1) {
    __shared__ uint4 bsm[2][N1 * BROW];   // W1[:, k0:k0+64] double-buffered, row n = 8 chunks of 8 bf16
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int lr = lane & 31, lh = lane >> 5;   // row/column within a 32-block, K half
    const int m0 = blockIdx.x * BM + 64 * wave;
    const uint8_t *abase = obs + (size_t)m0 * K1;     // wave-uniform base, 32-bit lane offsets
    const int rows_left = M - m0;
    floatx16 acc[2][8];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 8; b++) acc[a][b] = floatx16{};
    uint2 va[2][4];
    uint4 vb[8];
    // A fragments of step k0 (rows 32a+lr of this wave, 8 bytes at k0+16s+8lh) and this
    // thread's share of the W1 slice (row t, eight 16-byte chunks)
    auto load = [&](int k0) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int k = k0 + 16 * q + 8 * lh;
#pragma unroll
            for (int a = 0; a < 2; a++) {
                const int r = 32 * a + lr;
                va[a][q] = k < K1 && r < rows_left ? *(const uint2 *)(abase + (uint32_t)(r * K1 + k)) : make_uint2(0u, 0u);
            }
        }
#pragma unroll
        for (int c = 0; c < 8; c++)
            vb[c] = k0 + 8 * c < K1 ? *(const uint4 *)(w1 + (uint32_t)(t * K1 + k0 + 8 * c)) : make_uint4(0u, 0u, 0u, 0u);
    };
    load(0);
#pragma unroll
    for (int c = 0; c < 8; c++) bsm[0][t * BROW + c] = vb[c];
    __syncthreads();
    for (int ks = 0; ks < KSTEPS; ks++) {
        const int cur = ks & 1;
        bf16x8 fa[2][4];
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int q = 0; q < 4; q++) fa[a][q] = widen8(va[a][q]);
        const bool more = ks + 1 < KSTEPS;
        if (more) load(KS * (ks + 1));   // next step's global loads overlap this step's MFMAs
        const uint4 *brow = &bsm[cur][lr * BROW + lh];
        bf16x8 fb[8], fn[8];
#pragma unroll
        for (int b = 0; b < 8; b++) fb[b] = __builtin_bit_cast(bf16x8, brow[32 * b * BROW]);
#pragma unroll
        for (int q = 0; q < 4; q++) {   // K sub-steps of 16; the next sub-step's W1 fragments load meanwhile
            if (q < 3) {
#pragma unroll
                for (int b = 0; b < 8; b++) fn[b] = __builtin_bit_cast(bf16x8, brow[32 * b * BROW + 2 * (q + 1)]);
            }
#pragma unroll
            for (int b = 0; b < 8; b++)
#pragma unroll
                for (int a = 0; a < 2; a++) acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[a][q], fb[b], acc[a][b], 0, 0, 0);
            if (q < 3) {
#pragma unroll
                for (int b = 0; b < 8; b++) fb[b] = fn[b];
            }
        }
        if (more) {
#pragma unroll
            for (int c = 0; c < 8; c++) bsm[cur ^ 1][t * BROW + c] = vb[c];
        }
        __syncthreads();
    }
    // D lane l of block (a, b): rows 32a + 8(r/4) + 4(l/32) + r%4, column 32b + l%32
#pragma unroll
    for (int b = 0; b < 8; b++) {
        const int col = 32 * b + lr;
        const float bias = __uint_as_float((uint32_t)b1[col] << 16);
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + 32 * a + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (row < M) h1[(size_t)row * N1 + col] = f_to_bf16(fmaxf(acc[a][b][r] + bias, 0.f));
            }
    }
}

}  // namespace d1t

extern "C" int d1_trunk1(const uint8_t *obs, int M, const void *w1, const void *b1, void *h1, void *stream) {
    if (M < 0 || (M > 0 && (!obs || !w1 || !b1 || !h1))) return D1_E_ARG;
    if ((uintptr_t)obs % 8 || (uintptr_t)w1 % 16) return D1_E_ARG;
    if (M == 0) return 0;
    hipLaunchKernelGGL(d1t::k_trunk1, dim3((M + d1t::BM - 1) / d1t::BM), dim3(256), 0, (hipStream_t)stream, obs, M,
                       (const uint16_t *)w1, (const uint16_t *)b1, (uint16_t *)h1);
    return (int)hipGetLastError();
}
