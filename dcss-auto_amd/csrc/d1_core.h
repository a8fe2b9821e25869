// d1hip core: device code shared by the environment, wait and learning-task kernels.
//
// Wave-uniform RNG (PCG32 / Philox counter mode), 80x70 LDS bitmaps (70 rows x 3
// dwords), the player view, the bit-parallel distance field, melee and monster
// pathing of gpu-d1/src/sim.h. Everything is force-inlined into the kernels that
// include it; nothing here allocates or keeps state.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/d1hip.h"

namespace d1 {

constexpr int W = 80, H = 70, N = 5600, RW = 3;   // 3 dwords per 80-bit row
constexpr int ROWS_WORDS = H * RW;                // 210
constexpr int BIG = 1 << 20;
constexpr int FAR = 1 << 20;    // layer of a cell the distance field does not reach

// A kernel that needs a float staging area once the BFS data is dead defines
// D1_STAGE_FLOATS before including this header; the area overlays the BFS bitmaps.
#ifndef D1_STAGE_FLOATS
#define D1_STAGE_FLOATS 1
#endif
struct Smem {
    uint32_t floor[ROWS_WORDS];
    uint32_t viewed[ROWS_WORDS];
    uint32_t occ[ROWS_WORDS];
    union {
        struct {
            uint32_t reach[ROWS_WORDS];
            uint32_t front[ROWS_WORDS];
            // BFS layer mod 3 of every reached cell as two bit planes: lay0 = layer % 3 == 1,
            // lay1 = layer % 3 == 2. Cells that BFS-neighbour each other differ by at most one
            // layer, so their layers mod 3 fix the sign of every comparison the monster rules make
            int32_t rowpre[72];   // inclusive per-row prefix counts (episode reset)
            uint32_t lay0[ROWS_WORDS];
            uint32_t lay1[ROWS_WORDS];
        };
        float stage[D1_STAGE_FLOATS];
        uint32_t orow[30];   // the observation's 15 window rows, two words each (write_obs)
    };
    uint32_t rq[24];   // the repair search's queue (packed entries)
    // the player view when a kernel keeps it in LDS (Ctx::view_lds), quadrant q in words 2q
    // (low) and 2q+1; 32-bit words keep the struct's alignment at 4 bytes, so that kernels
    // that embed it do not grow (a one-wave workgroup at 10,240 B fits 16 to a CU)
    uint32_t vis[8];
};

// ---------------------------------------------------------------- small helpers
__device__ __forceinline__ int lane_id() { return (int)threadIdx.x; }
__device__ __forceinline__ int imin(int a, int b) { return a < b ? a : b; }
__device__ __forceinline__ int imax(int a, int b) { return a > b ? a : b; }
__device__ __forceinline__ int iabs(int a) { return a < 0 ? -a : a; }
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int lane_val(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ uint64_t ballot(bool b) { return __ballot(b); }
// DPP lane moves (GFX9 data-parallel primitives, no LDS round trip). `id` fills the lanes
// whose source is outside the wave or outside the written rows.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ int dpp(int v, int id) { return __builtin_amdgcn_update_dpp(id, v, CTRL, ROWS, 0xF, false); }
constexpr int DPP_QUAD_1032 = 0xB1, DPP_QUAD_2301 = 0x4E, DPP_ROW_HALF_MIRROR = 0x141, DPP_ROW_MIRROR = 0x140,
              DPP_ROW_BCAST15 = 0x142, DPP_ROW_BCAST31 = 0x143, DPP_WAVE_SHL1 = 0x130, DPP_WAVE_SHR1 = 0x138;
// lane l <- l-1 / l+1; bound control makes lane 0 / lane 63 (no source lane) read 0
__device__ __forceinline__ uint32_t lane_up(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, DPP_WAVE_SHR1, 0xF, 0xF, true);
}
__device__ __forceinline__ uint32_t lane_dn(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, DPP_WAVE_SHL1, 0xF, 0xF, true);
}
// Whole-wave reductions (every lane active): pairs, quads, half rows and rows by lane
// permutations, then row 0 into row 1 and row 2 into row 3 (row_bcast:15), rows 0-1 into
// rows 2-3 (row_bcast:31); lane 63 ends with the wave's result.
template <typename Op>
__device__ __forceinline__ int wave_reduce(int v, int id, Op op) {
    v = op(v, dpp<DPP_QUAD_1032>(v, id));
    v = op(v, dpp<DPP_QUAD_2301>(v, id));
    v = op(v, dpp<DPP_ROW_HALF_MIRROR>(v, id));
    v = op(v, dpp<DPP_ROW_MIRROR>(v, id));
    v = op(v, dpp<DPP_ROW_BCAST15, 0xA>(v, id));
    v = op(v, dpp<DPP_ROW_BCAST31, 0xC>(v, id));
    return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ int wave_max(int v) {
    return wave_reduce(v, (int)0x80000000, [](int a, int b) { return imax(a, b); });
}
__device__ __forceinline__ int wave_min(int v) {
    return wave_reduce(v, 0x7FFFFFFF, [](int a, int b) { return imin(a, b); });
}
__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
    return (uint32_t)wave_reduce((int)v, 0, [](int a, int b) { return (int)((uint32_t)a + (uint32_t)b); });
}
// gpu-d1/src/sim.h:14
__device__ __forceinline__ int cheb(int a, int b) { return imax(iabs(a % W - b % W), iabs(a / W - b / W)); }
// the same for two cells of the map (0 <= a, b < N): unsigned division by the width is shorter
__device__ __forceinline__ int cheb_u(int a, int b) {
    const uint32_t ua = (uint32_t)a, ub = (uint32_t)b;
    return imax(iabs((int)(ua % W) - (int)(ub % W)), iabs((int)(ua / W) - (int)(ub / W)));
}
// gpu-d1/src/sim.h:201-206: N, E, S, W, NE, SE, SW, NW
__device__ __forceinline__ int nbr(int p, int d) {
    int ddx = d == 1 || d == 4 || d == 5 ? 1 : d == 3 || d == 6 || d == 7 ? -1 : 0;
    int ddy = d == 0 || d == 4 || d == 7 ? -1 : d == 2 || d == 5 || d == 6 ? 1 : 0;
    int x = p % W + ddx, y = p / W + ddy;
    return x >= 0 && x < W && y >= 0 && y < H ? y * W + x : -1;
}
__device__ __forceinline__ bool inb(int x, int y) { return x >= 0 && x < W && y >= 0 && y < H; }
__device__ __forceinline__ bool bit_at(const uint32_t *bm, int x, int y) {
    return (bm[y * RW + (x >> 5)] >> (x & 31)) & 1u;
}
__device__ __forceinline__ bool bit(const uint32_t *bm, int p) { return bit_at(bm, p % W, p / W); }

struct Row {
    uint32_t a, b, c;   // bits 0-31, 32-63, 64-79
};
__device__ __forceinline__ Row row_ld(const uint32_t *bm, int y) { return {bm[y * RW], bm[y * RW + 1], bm[y * RW + 2]}; }
__device__ __forceinline__ void row_st(uint32_t *bm, int y, Row r) { bm[y * RW] = r.a; bm[y * RW + 1] = r.b; bm[y * RW + 2] = r.c; }
__device__ __forceinline__ Row row_or(Row x, Row y) { return {x.a | y.a, x.b | y.b, x.c | y.c}; }
__device__ __forceinline__ Row row_and(Row x, Row y) { return {x.a & y.a, x.b & y.b, x.c & y.c}; }
__device__ __forceinline__ Row row_andn(Row x, Row y) { return {x.a & ~y.a, x.b & ~y.b, x.c & ~y.c}; }
__device__ __forceinline__ Row row_shl1(Row r) { return {r.a << 1, (r.b << 1) | (r.a >> 31), ((r.c << 1) | (r.b >> 31)) & 0xFFFFu}; }
__device__ __forceinline__ Row row_shr1(Row r) { return {(r.a >> 1) | (r.b << 31), (r.b >> 1) | (r.c << 31), r.c >> 1}; }
__device__ __forceinline__ bool row_any(Row r) { return (r.a | r.b | r.c) != 0; }
__device__ __forceinline__ int row_popc(Row r) { return __popc(r.a) + __popc(r.b) + __popc(r.c); }
// bits [x0, x1] of the 32-bit word starting at bit `base`
__device__ __forceinline__ uint32_t word_range(int x0, int x1, int base) {
    int lo = imax(x0 - base, 0), hi = imin(x1 - base, 31);
    return lo > hi ? 0u : ((hi == 31 ? 0xFFFFFFFFu : ((1u << (hi + 1)) - 1u)) & ~((1u << lo) - 1u));
}
// bits [x0, x1] (inclusive, clipped to 0..79)
__device__ __forceinline__ Row row_range(int x0, int x1) {
    x0 = imax(x0, 0);
    x1 = imin(x1, W - 1);
    if (x0 > x1) return Row{0, 0, 0};
    return Row{word_range(x0, x1, 0), word_range(x0, x1, 32), word_range(x0, x1, 64) & 0xFFFFu};
}
// 15-bit window pattern v (bit k = x px-7+k) placed on an 80-bit row
__device__ __forceinline__ Row row_place15(uint32_t v, int px) {
    int shift = px - 7;
    uint64_t lo, hi;
    if (shift < 0) { lo = (uint64_t)v >> (-shift); hi = 0; }
    else if (shift < 64) { lo = (uint64_t)v << shift; hi = shift ? ((uint64_t)v >> (64 - shift)) : 0; }
    else { lo = 0; hi = (uint64_t)v << (shift - 64); }
    return {(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi & 0xFFFFu};
}
// position of the j-th set bit (j < popc(v))
__device__ __forceinline__ int select32(uint32_t v, int j) {
    int pos = 0;
    for (int s = 16; s; s >>= 1) {
        int c = __popc(v & ((1u << s) - 1u));
        if (j >= c) { j -= c; v >>= s; pos += s; }
    }
    return pos;
}
// position of the k-th set bit of a 64-bit mask (k < popcount)
__device__ __forceinline__ int select64(uint64_t m, int k) {
    int lo = __popc((uint32_t)m);
    return k < lo ? select32((uint32_t)m, k) : 32 + select32((uint32_t)(m >> 32), k - lo);
}
__device__ __forceinline__ int row_select(Row r, int j) {
    int c0 = __popc(r.a);
    if (j < c0) return select32(r.a, j);
    j -= c0;
    int c1 = __popc(r.b);
    if (j < c1) return 32 + select32(r.b, j);
    return 64 + select32(r.c, j - c1);
}
__device__ __forceinline__ uint32_t fmix32(uint32_t h) {
    h ^= h >> 16; h *= 0x85ebca6bu; h ^= h >> 13; h *= 0xc2b2ae35u; h ^= h >> 16;
    return h;
}
__device__ __forceinline__ uint32_t term(uint32_t word, uint32_t index) { return fmix32(word ^ (index * 0x9E3779B9u)); }
__device__ __forceinline__ uint64_t mix64(uint64_t x) {   // gpu-d1/src/sim.h:15-20
    x += 0x9e3779b97f4a7c15ULL;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ULL;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebULL;
    return x ^ (x >> 31);
}

// ---------------------------------------------------------------- RNG (wave-uniform)
// PCG32 XSH-RR as gpu-d1/src/sim.h:21-60, or Philox4x32-10 where draw k of stream
// (t, env, domain) is word k%4 of Philox(ctr={k/4, t, env, domain}, key=seed).
//
// The stream is consumed through a 64-lane buffer: lane l of `buf` holds draw base+l,
// refilled 64 draws at a time by one vector computation (PCG by jump-ahead from the
// table below, Philox one counter per lane), so a draw is one readlane and the refill
// code exists once per kernel instead of at every draw site.

// PCG jump-ahead: state after j steps = A[j]*s + C[j]*inc (A[j] = a^j, C[j] = sum_{i<j} a^i).
struct PcgJump {
    uint64_t a[65], c[65];
    constexpr PcgJump() : a(), c() {
        a[0] = 1; c[0] = 0;
        for (int j = 1; j <= 64; j++) { a[j] = a[j - 1] * 6364136223846793005ULL; c[j] = c[j - 1] * 6364136223846793005ULL + 1; }
    }
};
__constant__ constexpr PcgJump kJump{};

__device__ __forceinline__ uint32_t pcg_out(uint64_t old) {
    uint32_t x = (uint32_t)(((old >> 18) ^ old) >> 27), r = (uint32_t)(old >> 59);
    return (x >> r) | (x << ((0u - r) & 31u));
}
// PCG32 output of the state `lane` steps after `st`.
__device__ __noinline__ uint32_t pcg_lane(uint64_t st, uint64_t inc, int lane) {
    return pcg_out(kJump.a[lane] * st + kJump.c[lane] * inc);
}
// Word idx%4 of Philox4x32-10(ctr = {idx/4, t, env, dom}, key = {key0, key1})
// (Salmon et al., SC'11: multipliers 0xD2511F53/0xCD9E8D57, Weyl increments
// 0x9E3779B9/0xBB67AE85).
__device__ __noinline__ uint32_t philox_lane(uint32_t key0, uint32_t key1, uint32_t t, uint32_t env, uint32_t dom,
                                             uint32_t idx) {
    uint32_t c0 = idx >> 2, c1 = t, c2 = env, c3 = dom, k0 = key0, k1 = key1;
#pragma unroll
    for (int r = 0; r < 10; r++) {
        uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
        uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
        uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
        k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
    }
    uint32_t j = idx & 3u;
    return j == 0 ? c0 : j == 1 ? c1 : j == 2 ? c2 : c3;
}

struct Rng {
    uint64_t st, inc;                   // PCG32: the state before draw `sb`
    uint32_t key0, key1, t, env, dom;   // counter stream
    uint32_t base, o;                   // lane l of buf holds draw base + l; the next draw is base + o
    uint32_t sb;                        // PCG state index
    uint32_t buf;
    int mode;

    __device__ __forceinline__ uint32_t k() const { return base + o; }   // index of the next draw
    // Draw values are a function of their index alone, so the buffer may be refilled at any
    // index: a fill that comes early changes no value.
    __device__ __forceinline__ void fill(uint32_t at) {
        int lane = (int)threadIdx.x;
        if (mode == 0) {
            uint32_t j = at - sb;   // <= 64: a fill happens at most 64 draws after the last one
            st = kJump.a[j] * st + kJump.c[j] * inc;
            sb = at;
            buf = pcg_lane(st, inc, lane);
        } else {
            buf = philox_lane(key0, key1, t, env, dom, at + (uint32_t)lane);
        }
        base = at;
        o = 0;
    }
    __device__ __forceinline__ uint32_t next() {
        if (o >= 64u) fill(base + o);
        uint32_t v = (uint32_t)__builtin_amdgcn_readlane((int)buf, (int)o);
        o++;
        return v;
    }
    // A rule that makes at most n draws reserves them: the buffer is refilled now if fewer
    // than n remain, and its draws (RES) skip the per-draw buffer check.
    __device__ __forceinline__ void reserve(uint32_t n) {
        if (o > 64u - n) fill(base + o);
    }
    template <bool RES>
    __device__ __forceinline__ uint32_t take() {
        if (RES) {
            uint32_t v = (uint32_t)__builtin_amdgcn_readlane((int)buf, (int)o);
            o++;
            return v;
        }
        return next();
    }
    // PCG32 state before draw k (what the sequential generator would hold now)
    __device__ __forceinline__ uint64_t pcg_state() const {
        uint32_t j = base + o - sb;
        return kJump.a[j] * st + kJump.c[j] * inc;
    }
    // gpu-d1/src/sim.h:36-51. Inside a reservation of n (RES), a rejected draw's redraws are
    // checked draws and the reservation is renewed after them.
    template <bool RES = false, uint32_t NRES = 0>
    __device__ __forceinline__ int r(int bound) {
        if (bound <= 1) return 0;
        uint32_t x = take<RES>();
        uint64_t m = (uint64_t)x * (uint32_t)bound;
        uint32_t low = (uint32_t)m;
        if (low < (uint32_t)bound) {
            uint32_t th = (0u - (uint32_t)bound) % (uint32_t)bound;
            while (low < th) {
                x = next();
                m = (uint64_t)x * (uint32_t)bound;
                low = (uint32_t)m;
            }
            if (RES) reserve(NRES);
        }
        return (int)(m >> 32);
    }
    template <bool RES = false, uint32_t NRES = 0>
    __device__ __forceinline__ int avg(int n) { int a = r<RES, NRES>(n); return (a + r<RES, NRES>(n + 1)) / 2; }   // sim.h:52-55
    template <bool RES = false, uint32_t NRES = 0>
    __device__ __forceinline__ int round(int n, int d) { int rem = n % d; return n / d + (rem && r<RES, NRES>(d) < rem); }  // sim.h:56-59
    __device__ __forceinline__ void pcg_load(uint64_t state, uint64_t increment) {
        mode = 0; st = state; inc = increment; sb = 0; base = 0u - 64u; o = 64;   // next draw 0, buffer empty
    }
    __device__ __forceinline__ void pcg_seed(uint64_t s, uint64_t seq) {   // sim.h:29-35: two steps around +s
        uint64_t i = (seq << 1) | 1;
        uint64_t v = i;   // 0 * a + inc
        v += s;
        v = v * 6364136223846793005ULL + i;
        pcg_load(v, i);
    }
    __device__ __forceinline__ void counter(uint64_t key, uint32_t e, uint32_t tt, uint32_t d) {
        mode = 1; key0 = (uint32_t)key; key1 = (uint32_t)(key >> 32); env = e; t = tt; dom = d;
        sb = 0; base = 0u - 64u; o = 64; st = 0; inc = 0;
    }
};

// Reservoir choice over `total` eligible cells: the 1-based count c is kept when
// r(c) == 0, the last kept count wins (gpu-d1/branches/d1-stairs-v2/src/learn.cu:432-441).
// 64 counts per pass: lane l evaluates count c0+l from the draw it would get if no
// earlier draw in the pass were rejected (the buffer refilled at the current index);
// a pass in which any Lemire rejection is possible (low < bound) is replayed serially,
// so the draw sequence is the serial one.
__device__ __forceinline__ int reservoir(Rng &s, int total, int lane) {
    int chosen = total >= 1 ? 0 : -1;
    int c0 = 2;
    while (c0 <= total) {
        int cnt = imin(64, total - c0 + 1);
        int c = c0 + lane;
        if (s.o != 0) s.fill(s.k());
        uint64_t m = (uint64_t)s.buf * (uint32_t)c;
        bool act = lane < cnt;
        bool risky = act && (uint32_t)m < (uint32_t)c;
        if (ballot(risky)) {
            for (int cc = c0; cc < c0 + cnt; cc++) if (s.r(cc) == 0) chosen = cc - 1;
        } else {
            uint64_t keep = ballot(act && (m >> 32) == 0);
            if (keep) chosen = c0 + 63 - __clzll((long long)keep) - 1;
            s.o += (uint32_t)cnt;
        }
        c0 += cnt;
    }
    return chosen;
}

// ---------------------------------------------------------------- world context
struct Ctx {
    Smem *sm;
    const D1Config *c;
    const uint64_t *rays;   // [nslots][64]
    int nslots;
    Rng g;
    int player, hp, regen, blocks, ticks, killed, decisions, floor_seen, episode, first_stair_tick, ncells;
    uint64_t stairs;   // three int16 cells at bits 0, 16, 32 (-1 = none)
    uint32_t t, env_id;
    // player view, quadrants (+,+) (-,+) (-,-) (+,-): bit 8*|dy| + |dx|. Kept in wave-uniform
    // registers, or in Smem::vis where a kernel sets view_lds (a constant per kernel): the
    // crowded step's monster phase holds enough live values that the registers spill.
    uint64_t visr[4];
    bool view_lds = false;
    // this lane's monster (lane < count)
    int mpos, mhp, menergy, mawake, mkind;
    int mlay;    // absolute BFS layer of the monster's cell (FAR when not known)
    // Stuck cache (kernels whose distance field depends on the player cell alone set
    // stuck_cache): mrad > 0 records that this lane's monster found no move with the player
    // on the current cell, and that the search behind that answer read no cell farther than
    // mrad (Chebyshev) from the monster. The answer stands while the player stays and no cell
    // within mrad changes occupancy (a move or a death there, or the monster's own move,
    // clears it), so the next act draws its rotation and waits without searching.
    int mrad = 0;
    bool stuck_cache = false;
    int lastl;   // last layer the field holds: a reached cell next to an unreached one is on it
    int lane;
    // distance-field memo in the state row (crowded layouts): its address, the player cell the
    // stored field belongs to (-1: none), and the player cell whose field LDS holds (-1: none)
    uint32_t *fcache = nullptr;
    int ftag = -1, fld = -1;
    bool rfloor = false;   // the memo's reach bitmap is the floor bitmap (not stored)
    // rows of the viewed bitmap changed since the world was loaded (vlo > vhi: none); the
    // default, every row, is what a world that was not loaded from a state row writes back
    int vlo = 0, vhi = H - 1;
};

// the four quadrant view masks (wave-uniform)
__device__ __forceinline__ void set_view(Ctx &x, uint64_t v0, uint64_t v1, uint64_t v2, uint64_t v3) {
    if (x.view_lds) {
        if (x.lane < 8) {
            const uint64_t v = x.lane < 2 ? v0 : x.lane < 4 ? v1 : x.lane < 6 ? v2 : v3;
            x.sm->vis[x.lane] = (uint32_t)(x.lane & 1 ? v >> 32 : v);
        }
        __syncthreads();
    } else {
        x.visr[0] = v0; x.visr[1] = v1; x.visr[2] = v2; x.visr[3] = v3;
    }
}
__device__ __forceinline__ uint64_t view_q(const Ctx &x, int q) {
    return x.view_lds ? (uint64_t)x.sm->vis[2 * q + 1] << 32 | x.sm->vis[2 * q] : x.visr[q];
}
__device__ __forceinline__ int stair_at(const Ctx &x, int k) { return (int16_t)(uint16_t)(x.stairs >> (16 * k)); }
__device__ __forceinline__ uint64_t pack_stairs(int a, int b, int c) {
    return (uint64_t)(uint16_t)a | (uint64_t)(uint16_t)b << 16 | (uint64_t)(uint16_t)c << 32;
}
__device__ __forceinline__ bool seen_at(const Ctx &x, int p) { return bit(x.sm->viewed, p) && bit(x.sm->floor, p); }

// 15x15 view lookup of the cell (dx, dy) from the player
__device__ __forceinline__ bool vis_rel(const Ctx &x, int dx, int dy) {
    if (iabs(dx) > 7 || iabs(dy) > 7) return false;
    int b = iabs(dy) * 8 + iabs(dx);
    uint64_t v = 0;
    if (dx >= 0 && dy >= 0) v |= view_q(x, 0);
    if (dx <= 0 && dy >= 0) v |= view_q(x, 1);
    if (dx <= 0 && dy <= 0) v |= view_q(x, 2);
    if (dx >= 0 && dy <= 0) v |= view_q(x, 3);
    return (v >> b) & 1;
}
// in_view, gpu-d1/branches/d1-stairs-v2/src/learn.cu:192-198 (terrain LOS, radius 7)
__device__ __forceinline__ bool in_view(const Ctx &x, int p) {
    if (p < 0) return false;
    return vis_rel(x, p % W - x.player % W, p / W - x.player / W);
}
__device__ __forceinline__ bool q_sx(int q) { return q == 0 || q == 3; }   // +x quadrants
__device__ __forceinline__ bool q_sy(int q) { return q < 2; }              // +y quadrants

// Opaque inside-blocker set of quadrant q around (ox, oy): lane j tests blocker
// (j%8, j/8) (gpu-d1/scripts/compile_fixture.py:35-39; out-of-bounds cells are clear).
__device__ __forceinline__ uint64_t opaque_set(const Ctx &x, int ox, int oy, int q) {
    int cx = ox + (q_sx(q) ? 1 : -1) * (x.lane & 7), cy = oy + (q_sy(q) ? 1 : -1) * (x.lane >> 3);
    bool op = inb(cx, cy) && !bit_at(x.sm->floor, cx, cy);
    return ballot(op);
}
// Player field of view: vis_q bit j set when target (j%8, j/8) of quadrant q is in
// bounds and one of its rays misses every opaque blocker.
// The ray slots are loaded four at a time, the next four in flight while the current ones
// are tested (past the last slot the loads repeat it, which changes no test): one load per
// slot, each waited for before the next, left the whole view waiting on 11 serial latencies.
__device__ __forceinline__ void compute_view(Ctx &x) {
    int px = x.player % W, py = x.player / W;
    const int ns = x.nslots;
    uint64_t m[4] = {0, 0, 0, 0};
    auto load4 = [&](int s0) {
#pragma unroll
        for (int i = 0; i < 4; i++) m[i] = x.rays[imin(s0 + i, ns - 1) * 64 + x.lane];
    };
    if (ns > 0) load4(0);   // in flight during the opaque-set reads
    uint64_t o0 = opaque_set(x, px, py, 0), o1 = opaque_set(x, px, py, 1);
    uint64_t o2 = opaque_set(x, px, py, 2), o3 = opaque_set(x, px, py, 3);
    bool a0 = false, a1 = false, a2 = false, a3 = false;
    for (int s0 = 0; s0 < ns; s0 += 4) {
        const uint64_t c0 = m[0], c1 = m[1], c2 = m[2], c3 = m[3];
        if (s0 + 4 < ns) load4(s0 + 4);
#define D1_RAY_TEST(v) a0 |= ((v) & o0) == 0; a1 |= ((v) & o1) == 0; a2 |= ((v) & o2) == 0; a3 |= ((v) & o3) == 0;
        D1_RAY_TEST(c0) D1_RAY_TEST(c1) D1_RAY_TEST(c2) D1_RAY_TEST(c3)
#undef D1_RAY_TEST
    }
    int tx = x.lane & 7, ty = x.lane >> 3;
    set_view(x, ballot(a0 && inb(px + tx, py + ty)), ballot(a1 && inb(px - tx, py + ty)),
             ballot(a2 && inb(px - tx, py - ty)), ballot(a3 && inb(px + tx, py - ty)));
}
// LOS from a monster to the player within Chebyshev 6 (monster_detects_player,
// gpu-d1/branches/d1-stairs-v2/src/learn.cu:199-207).
__device__ __forceinline__ bool detects(Ctx &x, int origin) {
    int ox = origin % W, oy = origin / W, dx = x.player % W - ox, dy = x.player / W - oy;
    if (iabs(dx) > 6 || iabs(dy) > 6) return false;
    if (!x.c->wake_los) return true;
    int t = iabs(dy) * 8 + iabs(dx);
    const bool has = x.lane < x.nslots;
    const uint64_t ray = has ? x.rays[x.lane * 64 + t] : 0;   // the same slot for every quadrant
    bool det = false;
    for (int q = 0; q < 4; q++) {
        bool sx = q_sx(q), sy = q_sy(q);
        if ((dx && (dx > 0) != sx) || (dy && (dy > 0) != sy)) continue;
        uint64_t opq = opaque_set(x, ox, oy, q);
        bool alive = has && (ray & opq) == 0;
        det |= ballot(alive) != 0;
    }
    return det;
}

// Reveal, gpu-d1/branches/d1-stairs-v2/src/learn.cu:298-333: viewed |= view; returns
// the number of floor cells seen for the first time (seen == viewed floor).
__device__ __forceinline__ int reveal(Ctx &x) {
    compute_view(x);
    int px = x.player % W, py = x.player / W;
    int fresh = 0;
    int dy = x.lane - 7, y = py + dy;
    bool mine = x.lane < 15 && y >= 0 && y < H;
    Row mask{0, 0, 0};
    if (mine) {
        int ay = iabs(dy);
        uint32_t R = 0, L = 0;
        if (dy >= 0) { R |= (uint32_t)(view_q(x, 0) >> (8 * ay)) & 0xFFu; L |= (uint32_t)(view_q(x, 1) >> (8 * ay)) & 0xFFu; }
        if (dy <= 0) { R |= (uint32_t)(view_q(x, 3) >> (8 * ay)) & 0xFFu; L |= (uint32_t)(view_q(x, 2) >> (8 * ay)) & 0xFFu; }
        uint32_t v15 = (__builtin_bitreverse32(L) >> 24) | (R << 7);
        mask = row_place15(v15, px);
        Row old = row_ld(x.sm->viewed, y);
        Row fl = row_ld(x.sm->floor, y);
        fresh = row_popc(row_and(row_andn(mask, old), fl));
    }
    __syncthreads();
    if (mine) row_st(x.sm->viewed, y, row_or(mask, row_ld(x.sm->viewed, y)));
    __syncthreads();
    x.vlo = imin(x.vlo, imax(py - 7, 0));
    x.vhi = imax(x.vhi, imin(py + 7, H - 1));
    int total = (int)wave_sum((uint32_t)fresh);
    x.floor_seen += total;
    return total;
}

__device__ __forceinline__ int stair_index(const Ctx &x) {
    for (int k = 0; k < 3; k++) if (stair_at(x, k) >= 0 && x.player == stair_at(x, k)) return k + 1;
    return 0;
}
__device__ __forceinline__ int known_stairs(const Ctx &x) {
    int n = 0;
    for (int k = 0; k < 3; k++) n += stair_at(x, k) >= 0 && seen_at(x, stair_at(x, k));
    return n;
}
__device__ __forceinline__ bool visible_awake(const Ctx &x) {
    bool me = x.lane < x.c->count && x.mhp > 0 && x.mawake && in_view(x, x.mpos);
    return ballot(me) != 0;
}
__device__ __forceinline__ void occ_set(Ctx &x, int p, bool on) {
    if (x.lane == 0) {
        uint32_t *w = &x.sm->occ[(p / W) * RW + ((p % W) >> 5)];
        uint32_t b = 1u << ((p % W) & 31);
        *w = on ? (*w | b) : (*w & ~b);
    }
    __syncthreads();
}

__device__ __forceinline__ void occ_set_lane(Ctx &x, int p) {
    atomicOr(&x.sm->occ[(p / W) * RW + ((p % W) >> 5)], 1u << ((p % W) & 31));
}
__device__ __forceinline__ void occ_clear_lane(Ctx &x, int p) {
    atomicAnd(&x.sm->occ[(p / W) * RW + ((p % W) >> 5)], ~(1u << ((p % W) & 31)));
}

// ---------------------------------------------------------------- cell selection
// Row prefix counts of a bitmap (rows in `bm`), stored inclusive in sm->rowpre.
__device__ __forceinline__ int row_prefix(Ctx &x, const uint32_t *bm) {
    int y0 = x.lane, y1 = x.lane + 64;
    int c0 = row_popc(row_ld(bm, y0));
    int c1 = y1 < H ? row_popc(row_ld(bm, y1)) : 0;
    int s0 = c0;
    for (int o = 1; o < 64; o <<= 1) { int v = __shfl_up(s0, o); if (x.lane >= o) s0 += v; }
    int tot0 = lane_val(s0, 63);
    int s1 = c1;
    for (int o = 1; o < 64; o <<= 1) { int v = __shfl_up(s1, o); if (x.lane >= o) s1 += v; }
    __syncthreads();
    x.sm->rowpre[y0] = s0;
    if (y1 < H) x.sm->rowpre[y1] = s1 + tot0;
    __syncthreads();
    return x.sm->rowpre[H - 1];
}
// The k-th set cell (row-major) of bitmap `bm`, given its rowpre.
__device__ __forceinline__ int select_cell(Ctx &x, const uint32_t *bm, int k) {
    int lo = 0, hi = H - 1;   // first row with rowpre > k
    while (lo < hi) { int mid = (lo + hi) >> 1; if (x.sm->rowpre[mid] > k) hi = mid; else lo = mid + 1; }
    int before = lo ? x.sm->rowpre[lo - 1] : 0;
    return lo * W + row_select(row_ld(bm, lo), k - before);
}

// ---------------------------------------------------------------- monsters
__device__ __forceinline__ int kind_speed(const D1Config *c, int k) {
    int s = c->kinds[0].speed;
    s = k == 1 ? c->kinds[1].speed : s;
    s = k == 2 ? c->kinds[2].speed : s;
    s = k == 3 ? c->kinds[3].speed : s;
    s = k == 4 ? c->kinds[4].speed : s;
    s = k == 5 ? c->kinds[5].speed : s;
    return s;
}
// gpu-d1/src/sim.h:130-163 (kind = the acting monster's kind)
__device__ __forceinline__ void attack(Ctx &x, int kind) {
    const D1Config *c = x.c;
    // every configuration value the attack may need, read before its first branch
    const D1Kind k = c->kinds[kind];
    const int ac100 = c->ac100, ev100 = c->ev100, sh100 = c->sh100, shield_limit = c->shield_limit;
    const int gdr0 = c->gdr[0], gdr1 = c->gdr[1];
    Rng &r = x.g;
    constexpr uint32_t ND = 15;   // the most draws an attack makes without a rejection
    r.reserve(ND);
    int hit = r.r<true, ND>(k.tohit + 1);
    int ev = r.round<true, ND>(ev100, 100);
    ev = r.avg<true, ND>(2 * ev);
    int margin = hit - ev;
    if (r.r<true, ND>(100) < 5) margin = (r.r<true, ND>(2) ? 1 : -1) * 1000;
    int bypass = r.r<true, ND>(k.bypass);
    int sh = r.round<true, ND>(sh100, 100);
    int block = r.avg<true, ND>(sh * 2) / 3 - 1;
    if (block >= bypass && x.blocks < shield_limit) { x.blocks++; return; }
    if (margin < 0) return;
    int damage = 1 + r.r<true, ND>(k.damage);
    int ac = r.round<true, ND>(ac100, 100);
    int gac = r.round<true, ND>(ac100, 100);
    int gdr = imin(imax(gac - ac100 / 100, 0), 1) ? gdr1 : gdr0;
    int saved = r.r<true, ND>(ac + 1);
    int half = r.round<true, ND>(ac, 2);
    saved = imax(saved, imin(gdr * k.damage / 100, half));
    damage = imax(0, damage - saved);
    x.hp -= damage;
}
// BFS layer mod 3 of cell q (meaningful where reach is set)
__device__ __forceinline__ int lay3(const Smem *sm, int q) { return (int)bit(sm->lay0, q) | ((int)bit(sm->lay1, q) << 1); }
// layer(q) - layer(r) from the layers mod 3 of two reached cells whose layers differ by at
// most one (8-neighbours on the BFS graph): -1, 0 or +1
__device__ __forceinline__ int step3(int mq, int mr) {
    const int d = mq - mr;
    return d == 1 || d == -2 ? 1 : (d == -1 || d == 2 ? -1 : 0);
}
__device__ __forceinline__ bool walkable(const Ctx &x, int q) {
    return q >= 0 && bit(x.sm->floor, q) && q != x.player && !bit(x.sm->occ, q);
}
// ---------------------------------------------------------------- monster moves in coordinates
// Direction d (N,E,S,W,NE,SE,SW,NW) as offsets: two bits of dx+1 / dy+1 per direction.
constexpr uint32_t DXP = 1u | 2u << 2 | 1u << 4 | 0u << 6 | 2u << 8 | 2u << 10 | 0u << 12 | 0u << 14;
constexpr uint32_t DYP = 0u | 1u << 2 | 2u << 4 | 1u << 6 | 0u << 8 | 2u << 10 | 2u << 12 | 0u << 14;
__device__ __forceinline__ int ddx(int d) { return (int)((DXP >> (2 * d)) & 3u) - 1; }
__device__ __forceinline__ int ddy(int d) { return (int)((DYP >> (2 * d)) & 3u) - 1; }
// The bitmap words of one cell (x, y): walkable (floor, unoccupied, not the player), reached
// by the distance field, its layer mod 3, queued by the repair search.
struct Cell {
    bool walk, reached, queued;
    int m3;
};
__device__ __forceinline__ Cell cell_at(const Smem *sm, int x, int y, int plx, int ply) {
    Cell c{false, false, false, 0};
    if ((unsigned)x >= (unsigned)W || (unsigned)y >= (unsigned)H) return c;
    const int w = y * RW + (x >> 5);
    const uint32_t b = 1u << (x & 31);
    c.walk = (sm->floor[w] & b) && !(sm->occ[w] & b) && !(x == plx && y == ply);
    c.reached = (sm->reach[w] & b) != 0;
    c.queued = (sm->front[w] & b) != 0;
    c.m3 = (int)((sm->lay0[w] & b) != 0) | ((int)((sm->lay1[w] & b) != 0) << 1);
    return c;
}

// The 24-node detour of gpu-d1/src/sim.h:227-252: a FIFO search from p over walkable cells
// in direction order N,E,S,W,NE,SE,SW,NW, queueing at most 24 cells; the first neighbour (in
// head, direction order) of a queued cell that is walkable and lower than p returns the
// first step towards it. Queue entries live in sm->rq, one packed word each (x, y, the
// first step's direction from p, layer mod 3, absolute layer or RQ_FAR); sm->front marks
// queued cells.
//
// Up to eight heads are expanded per pass (lane = 8 x head offset + direction), which is the
// sequential order: heads appended during a pass come after every head of the pass, a lower
// cell is never queued (it would have returned), and a candidate that also neighbours an
// earlier head of the pass is that head's to append (it enumerates all eight neighbours and
// sees the same queued set), so the first occurrences in lane order are appended, in order,
// while the queue has room. Layers are exact along the queue: a reached neighbour of a
// reached cell is one of -1/0/+1 away, which the layers mod 3 decide; a reached neighbour of
// an unreached cell is on the field's last layer; an unreached cell lies beyond every layer
// that could be lower than p.
constexpr int REPAIR_Q = 24, RQ_FAR = 8191;
static_assert(REPAIR_Q <= (int)(sizeof(Smem::rq) / sizeof(uint32_t)), "the queue fits Smem::rq");
__device__ __forceinline__ uint32_t rq_pack(int x, int y, int fdir, int m3, int lay) {
    return (uint32_t)x | (uint32_t)y << 7 | (uint32_t)fdir << 14 | (uint32_t)m3 << 17 | (uint32_t)imin(lay, RQ_FAR) << 19;
}
__device__ __forceinline__ int next_layer(const Cell &c, int hlay, int hm, int lastl) {
    if (!c.reached) return RQ_FAR;
    return hlay < RQ_FAR ? hlay + step3(c.m3, hm) : lastl;
}
// Returns the first step's direction from p (-1: none); with -1, rad is the largest Chebyshev
// distance from p of a cell the search read (its queued cells' neighbours).
__device__ __forceinline__ int repair_search(Ctx &x, int px, int py, int plx, int ply, int mp, int plag, int &rad) {
    Smem *sm = x.sm;
    const int hoff = x.lane >> 3, dir = x.lane & 7, dx = ddx(dir), dy = ddy(dir);
    const int lastl = imin(x.lastl, RQ_FAR - 1);
    if (x.lane == 0) {
        sm->rq[0] = rq_pack(px, py, 0, mp, plag);
        sm->front[py * RW + (px >> 5)] |= 1u << (px & 31);
    }
    __syncthreads();
    int len = 1, head = 0, result = -1;
    while (head < len && len < REPAIR_Q) {
        const int nh = imin(8, len - head), h = head + hoff;
        const uint32_t hw = sm->rq[imin(h, REPAIR_Q - 1)];
        const int hx = (int)(hw & 127u), hy = (int)((hw >> 7) & 127u), hf = (int)((hw >> 14) & 7u);
        const int hm = (int)((hw >> 17) & 3u), hlay = (int)(hw >> 19);
        const bool hv = hoff < nh;
        const int nx = hx + dx, ny = hy + dy;
        const Cell c = hv ? cell_at(sm, nx, ny, plx, ply) : Cell{false, false, false, 0};
        const int nlay = c.walk ? next_layer(c, hlay, hm, lastl) : RQ_FAR;
        const int fdir = h == 0 ? dir : hf;
        const uint64_t lm = ballot(c.walk && nlay < plag);
        if (lm) {
            result = lane_val(fdir, __ffsll((unsigned long long)lm) - 1);
            break;
        }
        bool cand = c.walk && !c.queued;
        for (int j = 0; j + 1 < nh; j++) {   // earlier heads of the pass own their neighbours
            const uint32_t jw = (uint32_t)lane_val((int)hw, 8 * j);
            const int ex = nx - (int)(jw & 127u), ey = ny - (int)((jw >> 7) & 127u);
            cand = cand && !(hoff > j && ex >= -1 && ex <= 1 && ey >= -1 && ey <= 1);
        }
        const uint64_t cm = ballot(cand);
        const int cnt = imin(__popcll(cm), REPAIR_Q - len);
        const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(cm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)cm, 0u));
        if (cand && rank < cnt) {
            sm->rq[len + rank] = rq_pack(nx, ny, fdir, c.m3, nlay);
            atomicOr(&sm->front[ny * RW + (nx >> 5)], 1u << (nx & 31));
        }
        len += cnt;
        head += nh;
        __syncthreads();
    }
    // Queue full: nothing more is appended and a queued cell is never lower, so the
    // remaining heads only look for the first lower neighbour, eight heads per pass.
    for (; result < 0 && head < len; head += 8) {
        const int h = head + hoff;
        const uint32_t hw = sm->rq[imin(h, REPAIR_Q - 1)];
        const int hx = (int)(hw & 127u), hy = (int)((hw >> 7) & 127u), hf = (int)((hw >> 14) & 7u);
        const int hm = (int)((hw >> 17) & 3u), hlay = (int)(hw >> 19);
        const Cell c = h < len ? cell_at(sm, hx + dx, hy + dy, plx, ply) : Cell{false, false, false, 0};
        const int nlay = c.walk ? next_layer(c, hlay, hm, lastl) : RQ_FAR;
        const uint64_t lm = ballot(c.walk && nlay < plag);
        if (lm) result = lane_val(h == 0 ? dir : hf, __ffsll((unsigned long long)lm) - 1);
    }
    int qd = 0;
    if (x.lane < len) {
        const uint32_t qw = sm->rq[x.lane];
        const int qx = (int)(qw & 127u), qy = (int)((qw >> 7) & 127u);
        atomicAnd(&sm->front[qy * RW + (qx >> 5)], ~(1u << (qx & 31)));
        qd = imax(iabs(qx - px), iabs(qy - py));
    }
    if (result < 0 && x.stuck_cache) rad = wave_max(qd) + 1;
    __syncthreads();
    return result;
}
// A sufficient test that the detour search finds nothing, without its queue. The search
// queues cells in breadth-first order from p over walkable cells, so the cells it queues
// lie within the first D rings around p, where D is the first ring that brings the count
// (p included) to REPAIR_Q, or the component's last ring. It succeeds only at a queued
// cell of layer plag with a walkable neighbour of layer plag - 1 (queued cells are never
// lower than p and neighbours differ by at most one layer), and that neighbour lies within
// ring D + 1. The rings are grown here as bitmaps of a 32 x 64 window (lane = row py-31+l,
// bit = column px-15+b), and every ringed cell is put in the classes of layer offset from
// plag it may have: 0, 1 or ">= 2" (p0, p1, g), from its layer mod 3 and the classes of its
// neighbours in earlier rings (a reached neighbour is one layer away at most; an unreached
// cell that p can walk to lies past the field's last layer, which is built ceil(speed/10)
// >= 2 layers past every mover's starting layer while a mover acts at most ceil(speed/10)
// times a turn and climbs at most one layer per act, so p is at least one layer below the
// last and that cell's offset is >= 2; the static and exhaustive fields reach every cell p
// can walk to): offset 0 needs a neighbour in 0 or 1, offset 1 any
// neighbour, ">= 2" a neighbour in ">= 2" (or in 1, for layer mod 3 == plag + 2). Until a
// cell can be lower than p the classes contain the true offsets, so a cell of layer mod 3 ==
// plag - 1 next to a possible offset 0 is the first place where a lower cell can appear.
// Returns true when rings 1..D+1 hold no such cell; false (run the search) when one may
// exist or the rings reach the window edge.
// On true, ring is the last ring grown: every cell the search would read lies within it.
__device__ __forceinline__ bool detour_ruled_out(const Ctx &x, int px, int py, int plx, int ply, int mp, int &ring) {
    const Smem *sm = x.sm;
    const int y = py - 31 + x.lane;
    // window bit b is column px-15+b; with a zero word prepended to the row, that is bit
    // vb+b of the widened row, vb = px+17 in 17..96: words j = vb/32 and j+1, shifted by vb%32
    const int vb = px + 17, j = vb >> 5, s = vb & 31;
    uint32_t fl = 0, oc = 0, re = 0, l0 = 0, l1 = 0;
    if ((unsigned)y < (unsigned)H) {
        // widened words j and j+1 are row words j-1 and j when those exist (j-1 >= 0, j <= 2);
        // the indices are clamped into the row so that every address read is in range
        const bool lo_in = j >= 1, hi_in = j <= RW - 1;
        const int wl = y * RW + imax(j - 1, 0), wh = y * RW + imin(j, RW - 1);
        auto win = [&](const uint32_t *bm) {
            const uint32_t lo = bm[wl], hw = bm[wh];
            return __builtin_amdgcn_alignbit(hi_in ? hw : 0u, lo_in ? lo : 0u, s);
        };
        fl = win(sm->floor);
        oc = win(sm->occ);
        re = win(sm->reach);
        l0 = win(sm->lay0);
        l1 = win(sm->lay1);
    }
    uint32_t walk = fl & ~oc;
    const int pb = plx - px + 15;
    if (x.lane == ply - py + 31 && (unsigned)pb < 32u) walk &= ~(1u << pb);
    // cells by layer offset class from p: layer mod 3 == mp, mp + 1, mp + 2 (reached cells)
    const uint32_t z = re & ~(l0 | l1);
    const uint32_t c0 = mp == 0 ? z : mp == 1 ? l0 : l1;
    const uint32_t c1 = mp == 0 ? l0 : mp == 1 ? l1 : z;
    const uint32_t c2 = mp == 0 ? l1 : mp == 1 ? z : l0;
    auto dil = [](uint32_t v) {
        const uint32_t h = v | (v << 1) | (v >> 1);
        return h | lane_up(h) | lane_dn(h);
    };
    uint32_t p0 = x.lane == 31 ? 1u << 15 : 0u, p1 = 0, g = 0, seen = p0;
    int count = 1;
    ring = 0;
    for (bool last = false;; ) {
        const uint32_t d0 = dil(p0), d1 = dil(p1), dg = dil(g);
        const uint32_t n = (d0 | d1 | dg) & walk & ~seen;
        ring++;
        if (ballot((n & c2 & d0) != 0)) return false;   // possibly lower than p
        const uint64_t rows = ballot(n != 0);
        if (!rows) return true;                         // the component ends
        if (last) return true;                          // ring D + 1 done
        // the next ring would leave the window: new cells in its first or last row or column
        if ((rows & 0x8000000000000001ull) || ballot((n & 0x80000001u) != 0)) return false;
        p0 |= n & c0 & (d0 | d1);
        p1 |= n & c1;   // every new cell neighbours an earlier one
        g |= n & (dg | (c2 & d1) | ~re);
        seen |= n;
        count += (int)wave_sum((uint32_t)__popc(n));
        last = count >= REPAIR_Q;                       // this was ring D
    }
}
// gpu-d1/src/sim.h:207-253: greedy descent with rotated order and 1/ties
// replacement, then a bounded 24-node BFS detour when stuck. p is a reached cell at
// absolute layer plag (every mover is reached before the field stops growing); the chosen
// cell's layer goes to qlag.
__device__ __forceinline__ int choose_move(Ctx &x, int id, int p, int plag, int &qlag) {
    int rotation = x.g.r(4);
    // A cached stuck answer stands for the whole choice: the player has not moved and no cell
    // within its radius (1 or more, so the eight neighbours too) changed occupancy, so no
    // neighbour is lower and the detour finds nothing, as when the answer was recorded.
    if (x.stuck_cache && lane_val(x.mrad, id) > 0) return -1;
    const Smem *sm = x.sm;
    const int px = (int)((uint32_t)p % W), py = (int)((uint32_t)p / W);
    const int plx = (int)((uint32_t)x.player % W), ply = (int)((uint32_t)x.player / W);
    const int mp = plag < FAR ? plag % 3 : 0;   // p's layer mod 3, as its bit planes hold it
    const int z = x.lane & 7;
    const int d = z < 4 ? (z + rotation) & 3 : 4 + ((z + rotation) & 3);
    const int nx = px + ddx(d), ny = py + ddy(d);
    const Cell c = x.lane < 8 ? cell_at(sm, nx, ny, plx, ply) : Cell{false, false, false, 0};
    const int q = ny * W + nx;
    // Reached neighbours differ from p by at most one layer, so only the lower ones can be
    // chosen: the first in rotated order is taken, each later one replaces it when
    // r(++ties) == 0. Equal, higher and unreached ones neither win nor draw.
    uint64_t low = ballot(c.walk && c.reached && step3(c.m3, mp) < 0);
    if (low) {
        int best = lane_val(q, __ffsll((unsigned long long)low) - 1), ties = 1;
        for (low &= low - 1; low; low &= low - 1) {
            int qq = lane_val(q, __ffsll((unsigned long long)low) - 1);
            if (x.g.r(++ties) == 0) best = qq;
        }
        qlag = plag - 1;
        return best;
    }
    // With no walkable neighbour the search would queue nothing after p and find nothing.
    if (!x.c->repair || !ballot(c.walk)) return -1;
    int rad = 0;
    if (detour_ruled_out(x, px, py, plx, ply, mp, rad)) {
        if (x.stuck_cache && x.lane == id) x.mrad = rad;
        return -1;
    }
    const int fd = repair_search(x, px, py, plx, ply, mp, imin(plag, RQ_FAR - 1), rad);
    if (fd < 0) {
        if (x.stuck_cache && x.lane == id) x.mrad = rad;
        return -1;
    }
    const int sx = px + ddx(fd), sy = py + ddy(fd);
    const Cell sc = cell_at(sm, sx, sy, plx, ply);   // a reached neighbour of p
    qlag = plag + step3(sc.m3, mp);
    return sy * W + sx;
}
// Bit-parallel BFS over floor from the player (the all-pairs row of
// gpu-d1/scripts/learn_env.py:31-39), stopped `margin` layers after every mover is reached.
// Lane l keeps rows l and (l < 6) 64+l of the frontier, reach, floor and the two layer-mod-3
// planes in registers; vertical neighbours arrive by DPP lane shifts, so a layer has no LDS
// access and no barrier. Reach and the planes are published to LDS at the end (the monster
// phase reads them); the frontier bitmap is left clear for the repair search's marks.
__device__ __forceinline__ Row row_up(Row r) { return {lane_up(r.a), lane_up(r.b), lane_up(r.c)}; }
__device__ __forceinline__ Row row_dn(Row r) { return {lane_dn(r.a), lane_dn(r.b), lane_dn(r.c)}; }
__device__ __forceinline__ Row row_lane(Row r, int l) {
    return {(uint32_t)lane_val((int)r.a, l), (uint32_t)lane_val((int)r.b, l), (uint32_t)lane_val((int)r.c, l)};
}
__device__ __forceinline__ Row row_sel(bool c, Row x, Row y) { return c ? x : y; }
__device__ __forceinline__ Row dilate(Row f, Row up, Row dn) {
    Row v = row_or(f, row_or(up, dn));
    return row_or(v, row_or(row_shl1(v), row_shr1(v)));
}
__device__ __forceinline__ void bfs(Ctx &x, uint64_t movers, int margin) {
    Smem *sm = x.sm;
    const int lane = x.lane;
    const bool has1 = lane < H - 64;
    const Row zero{0, 0, 0};
    // the movers' cells as bit rows, staged through the (cleared) frontier bitmap
    row_st(sm->front, lane, zero);
    if (has1) row_st(sm->front, 64 + lane, zero);
    __syncthreads();
    if ((movers >> lane) & 1) atomicOr(&sm->front[(x.mpos / W) * RW + ((x.mpos % W) >> 5)], 1u << ((x.mpos % W) & 31));
    __syncthreads();
    const Row mv0 = row_ld(sm->front, lane), mv1 = has1 ? row_ld(sm->front, 64 + lane) : zero;
    __syncthreads();
    row_st(sm->front, lane, zero);
    if (has1) row_st(sm->front, 64 + lane, zero);
    const Row fl0 = row_ld(sm->floor, lane), fl1 = has1 ? row_ld(sm->floor, 64 + lane) : zero;
    const int py = x.player / W, px = x.player % W;
    const Row pbit = row_range(px, px);
    Row f0 = lane == py ? pbit : zero, f1 = has1 && 64 + lane == py ? pbit : zero;
    Row r0 = f0, r1 = f1;
    Row a0 = zero, a1 = zero, b0 = zero, b1 = zero;   // layer % 3 == 1, layer % 3 == 2
    // a mover lane learns its cell's layer when a layer first covers it: its row is held by
    // lane (row & 63), whose newly reached mover bits are read out once per such lane
    const bool mover = (movers >> lane) & 1;
    const int my = mover ? x.mpos / W : 0, mword = mover ? (x.mpos % W) >> 5 : 0;
    const uint32_t mbit = mover ? 1u << ((x.mpos % W) & 31) : 0u;
    x.mlay = FAR;
    int m3 = 0, stop = 1 << 30, last = 0;
    for (int layer = 1; layer < N; layer++) {
        m3 = m3 == 2 ? 0 : m3 + 1;
        const Row f0_63 = row_lane(f0, 63);
        Row n0, n1 = zero;
        if (row_any(f0_63) || ballot(row_any(f1))) {   // rows 64.. can grow this layer
            const Row f1_0 = row_lane(f1, 0);
            const Row u0 = row_sel(lane == 0, zero, row_up(f0)), d0 = row_sel(lane == 63, f1_0, row_dn(f0));
            const Row u1 = row_sel(lane == 0, f0_63, row_up(f1)), d1 = row_sel(lane >= H - 65, zero, row_dn(f1));
            n0 = row_andn(row_and(dilate(f0, u0, d0), fl0), r0);
            n1 = has1 ? row_andn(row_and(dilate(f1, u1, d1), fl1), r1) : zero;
        } else {   // no frontier in rows 63..: the second row set neither grows nor feeds row 63
            const Row u0 = row_sel(lane == 0, zero, row_up(f0)), d0 = row_sel(lane == 63, zero, row_dn(f0));
            n0 = row_andn(row_and(dilate(f0, u0, d0), fl0), r0);
        }
        if (!ballot(row_any(n0) || row_any(n1))) break;
        last = layer;
        r0 = row_or(r0, n0); r1 = row_or(r1, n1);
        f0 = n0; f1 = n1;
        if (m3 == 1) { a0 = row_or(a0, n0); a1 = row_or(a1, n1); }
        if (m3 == 2) { b0 = row_or(b0, n0); b1 = row_or(b1, n1); }
        const Row h0 = row_and(n0, mv0), h1 = row_and(n1, mv1);
        for (uint64_t hit = ballot(row_any(h0) || row_any(h1)); hit; hit &= hit - 1) {
            const int l = __ffsll((unsigned long long)hit) - 1;
            const Row g = my >= 64 ? row_lane(h1, l) : row_lane(h0, l);
            const uint32_t w = mword == 0 ? g.a : mword == 1 ? g.b : g.c;
            if (mover && (my & 63) == l && (w & mbit)) x.mlay = layer;
        }
        if (stop == (1 << 30) && !ballot(row_any(row_andn(mv0, r0)) || row_any(row_andn(mv1, r1)))) stop = layer + margin;
        if (layer >= stop) break;
    }
    x.lastl = last;
    row_st(sm->reach, lane, r0);
    row_st(sm->lay0, lane, a0);
    row_st(sm->lay1, lane, b0);
    if (has1) { row_st(sm->reach, 64 + lane, r1); row_st(sm->lay0, 64 + lane, a1); row_st(sm->lay1, 64 + lane, b1); }
    __syncthreads();
}
// Cells a and b changed occupancy: stuck answers whose search read either are dropped.
__device__ __forceinline__ void stuck_touch(Ctx &x, int a, int b) {
    if (x.mrad > 0 && (cheb_u(x.mpos, a) <= x.mrad || cheb_u(x.mpos, b) <= x.mrad)) x.mrad = 0;
}
// gpu-d1/src/sim.h:254-269
// The mover's absolute layer follows it (the cell it steps to is a reached neighbour).
__device__ __forceinline__ void act(Ctx &x, int id) {
    if (x.lane == id) x.menergy -= 10;
    int p = lane_val(x.mpos, id);
    if (cheb_u(p, x.player) == 1) { attack(x, lane_val(x.mkind, id)); return; }
    int qlag = FAR;
    int q = choose_move(x, id, p, lane_val(x.mlay, id), qlag);
    if (q >= 0) {
        if (x.lane == 0) {   // occupancy follows the monster (one lane, then a wave-wide wait)
            const uint32_t up = (uint32_t)p, uq = (uint32_t)q;
            atomicAnd(&x.sm->occ[(up / W) * RW + ((up % W) >> 5)], ~(1u << ((up % W) & 31)));
            atomicOr(&x.sm->occ[(uq / W) * RW + ((uq % W) >> 5)], 1u << ((uq % W) & 31));
        }
        if (x.stuck_cache) stuck_touch(x, p, q);   // the mover's own entry too (p is its cell)
        __syncthreads();
        if (x.lane == id) { x.mpos = q; x.mlay = qlag; }
    }
}

}  // namespace d1
