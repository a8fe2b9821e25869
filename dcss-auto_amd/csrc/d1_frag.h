// d1hip: MFMA operand helpers shared by the policy forward (d1_forward.hip) and the PPO step
// (d1_ppo.hip), gfx950.
//
// MFMA: v_mfma_f32_32x32x16_bf16. Lane layouts (checked on the hardware): A lane l holds
// A[l%32][8(l/32)+j], B lane l holds B[8(l/32)+j][l%32], D lane l holds
// D[8(r/4)+4(l/32)+r%4][l%32]. The contraction order inside a 64-wide K chunk is free as
// long as A and B agree, so in chunk c, step q, slot j of a lane in half h stands for
// k = 64c + 32h + 8q + j: each lane then reads 32 contiguous K values per operand row.
//
// Fragment order. An operand that the MFMAs read as [row][k] (32-row block b, K chunk c,
// step q) is stored so that the 64 lanes' 16-byte pieces of one step are one contiguous
// kilobyte: element (row, k) at ((((b * nchunks + c) * 4 + q) * 64 + row%32 + 32h) * 8 + j).
// Every operand load is then one fully used 1 KB span instead of 32 rows x 32 bytes.
#ifndef D1_FRAG_H
#define D1_FRAG_H
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace d1f {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16;
// register-resident 8- and 16-byte pieces (HIP's uint2/uint4 structs, copied whole through
// references, can be left in scratch by the compiler; native vectors are not)
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Reductions over the 16 lanes of a DPP row (lane moves on the VALU instead of the LDS
// crossbar __shfl_xor goes through), combining partners in the order of the __shfl_xor
// butterfly with offsets 8, 4, 2, 1 and giving its results bit for bit: row_ror:8 is xor 8
// within a row; after that step lanes l and l^8 hold equal values, so row_ror:4 reads one
// holding lane l^4's value; quad_perm [2,3,0,1] and [1,0,3,2] are xor 2 and xor 1.
constexpr int DPP_ROR8 = 0x128, DPP_ROR4 = 0x124, DPP_XOR2 = 0x4E, DPP_XOR1 = 0xB1;
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_f<DPP_ROR8>(x);
    x += dpp_f<DPP_ROR4>(x);
    x += dpp_f<DPP_XOR2>(x);
    return x + dpp_f<DPP_XOR1>(x);
}
__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp_f<DPP_ROR8>(x));
    x = fmaxf(x, dpp_f<DPP_ROR4>(x));
    x = fmaxf(x, dpp_f<DPP_XOR2>(x));
    return fmaxf(x, dpp_f<DPP_XOR1>(x));
}

// x + (x of lane l ^ 32) and x + (x of lane l ^ 16), bit for bit as with __shfl_xor (the
// sum is commutative), through gfx950's lane-swap moves instead of the LDS crossbar:
// v_permlane32_swap with x as both operands returns x's low half in every lane of its first
// result and x's high half in every lane of its second (checked on the hardware);
// v_permlane16_swap does the same for the even and odd 16-lane rows of each half.
__device__ __forceinline__ float xor32_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_sum(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float bf(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }
// float -> bf16, round to nearest even; NaNs stay NaN (quiet bit set when the dropped half
// held the payload). Branch-free: in the epilogues this runs on hundreds of values per lane.
__device__ __forceinline__ uint16_t rb(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
    const uint32_t n = (u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u);
    return (uint16_t)((u & 0x7F800000u) == 0x7F800000u ? n : r);
}
// the same for inputs known not to be NaN (ReLU outputs: fmaxf(x, 0) never returns NaN);
// +-inf round to themselves
__device__ __forceinline__ uint16_t rb_num(float f) {
    const uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
// two bytes of x (at bit 8s) -> two bf16 in one dword (exact: byte values need 8 bits)
__device__ __forceinline__ uint32_t widen2(uint32_t x, int s) {   // one v_perm pairs the high halves
    const uint32_t lo = __float_as_uint((float)((x >> (8 * s)) & 255u));
    const uint32_t hi = __float_as_uint((float)((x >> (8 * s + 8)) & 255u));
    return __builtin_amdgcn_perm(hi, lo, 0x07060302u);
}
// four bytes -> four bf16 (exact): the high halves of the converted floats, paired by v_perm
// two floats -> two bf16 in one dword (lo in bits 0-15) with the hardware pack
// (v_cvt_pk_bf16_f32): round to nearest even, equal to rb() / rb_num() for every non-NaN
// input (checked on the hardware over all denormals, ties, infinities and a 1/257
// sample of all finite patterns); NaN in gives a quiet NaN.
__device__ __forceinline__ uint32_t cvt2(float lo, float hi) {
    typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
    const bf16x2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint2 widen4(uint32_t x) {
    const uint32_t f0 = __float_as_uint((float)(x & 255u)), f1 = __float_as_uint((float)((x >> 8) & 255u));
    const uint32_t f2 = __float_as_uint((float)((x >> 16) & 255u)), f3 = __float_as_uint((float)(x >> 24));
    return make_uint2(__builtin_amdgcn_perm(f1, f0, 0x07060302u), __builtin_amdgcn_perm(f3, f2, 0x07060302u));
}
__device__ __forceinline__ bf16x8 widen8(uint32_t x0, uint32_t x1) {
    return __builtin_bit_cast(bf16x8, make_uint4(widen2(x0, 0), widen2(x0, 2), widen2(x1, 0), widen2(x1, 2)));
}
__device__ __forceinline__ bf16x8 as_bf(uint4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ bf16x8 as_bf(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ floatx16 mfma(bf16x8 a, bf16x8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// D row of accumulator register r in lane half h
__device__ __forceinline__ int drow(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }
// fragment-order index of element (row, k) of a [rows][nch*64] bf16 operand
__device__ __forceinline__ size_t fidx(int row, int k, int nch) {
    return ((((size_t)(row >> 5) * nch + (k >> 6)) * 4 + ((k >> 3) & 3)) * 64 + (row & 31) + 32 * ((k >> 5) & 1)) * 8 +
           (k & 7);
}

}  // namespace d1f
#endif
