// d1hip: batched DCSS D:1 environment for MI355X (gfx950).
//
// One wavefront (64 lanes, one workgroup) owns one world per launch. The world's
// bitmaps (floor, viewed, living-monster occupancy, BFS reach/frontier) live in LDS
// as 70 rows x 3 dwords (12-byte stride, bank-conflict free for row-per-lane
// access); monster i lives in lane i's registers; the player, the RNG and the
// scalars are wave-uniform. Parallel pieces:
//   * field of view: lane j = blocker/target (x=j%8, y=j/8) of a quadrant; a ballot
//     gives the quadrant's opaque set, each lane tests its target's rays against it,
//     a second ballot gives the visible set (64 lanes = the 8x8 quadrant exactly);
//   * distance-from-player field: bit-parallel BFS over floor rows (lane = row),
//     stopped two layers after the farthest monster that will move this turn;
//   * scheduler: wave max-reduce of energy*128+127-id (the key of
//     gpu-d1/src/bench.cu:66-74); melee and RNG draws run in uniform code;
//   * observation: lane = window cell, one 8-byte store per cell (channel-last).
// Rules follow gpu-d1/src/sim.h and gpu-d1/branches/d1-stairs-v2/src/learn.cu;
// each function cites the lines it implements. Built with -ffp-contract=off so the
// reward arithmetic rounds exactly like the host's.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/d1hip.h"

namespace d1 {

constexpr int W = 80, H = 70, N = 5600, RW = 3;   // 3 dwords per 80-bit row
constexpr int ROWS_WORDS = H * RW;                // 210
constexpr int BIG = 1 << 20;

// ---------------------------------------------------------------- state row layout
struct Hdr {
    uint64_t rng_state;    // PCG state, or the 64-bit Philox key in counter mode
    uint64_t rng_inc;      // PCG increment (2*(env+1)+1)
    uint32_t env_id;
    uint32_t t;            // steps taken (counter-mode stream index)
    int32_t episode;
    int16_t player, hp, regen, ncells;
    int32_t ticks, killed, decisions, floor_seen;
    int16_t stairs[3];
    int16_t blocks;
    int32_t first_stair_tick;
};
static_assert(sizeof(Hdr) == 64, "header layout");
struct Mon {
    int16_t pos, hp, energy;
    uint8_t awake, kind;
};
static_assert(sizeof(Mon) == 8, "monster layout");

__host__ __device__ constexpr int off_viewed(int m) { return 64 + 8 * m; }
__host__ __device__ constexpr int off_floor(int m) { return off_viewed(m) + ROWS_WORDS * 4; }
__host__ __device__ constexpr int off_cells(int m) { return off_floor(m) + ROWS_WORDS * 4; }
__host__ __device__ constexpr int state_bytes(int m) { return (off_cells(m) + ROWS_WORDS * 4 + 63) / 64 * 64; }

struct Smem {
    uint32_t floor[ROWS_WORDS];
    uint32_t viewed[ROWS_WORDS];
    uint32_t occ[ROWS_WORDS];
    uint32_t reach[ROWS_WORDS];
    uint32_t front[ROWS_WORDS];
    union {
        uint8_t dist[N];        // BFS layer mod 256, valid where `reach` is set (monster phase)
        struct {
            uint32_t win[225];  // observation window: kind+1 | hp<<8 | stair<<16 (observation)
            int32_t rowpre[72]; // inclusive per-row prefix counts (episode reset)
        };
    };
};

// ---------------------------------------------------------------- small helpers
__device__ __forceinline__ int lane_id() { return (int)threadIdx.x; }
__device__ __forceinline__ int imin(int a, int b) { return a < b ? a : b; }
__device__ __forceinline__ int imax(int a, int b) { return a > b ? a : b; }
__device__ __forceinline__ int iabs(int a) { return a < 0 ? -a : a; }
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int lane_val(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ uint64_t ballot(bool b) { return __ballot(b); }
__device__ __forceinline__ int wave_max(int v) {
    for (int o = 32; o; o >>= 1) v = imax(v, __shfl_xor(v, o));
    return uni(v);
}
__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
    for (int o = 32; o; o >>= 1) v += (uint32_t)__shfl_xor((int)v, o);
    return (uint32_t)uni((int)v);
}
// gpu-d1/src/sim.h:14
__device__ __forceinline__ int cheb(int a, int b) { return imax(iabs(a % W - b % W), iabs(a / W - b / W)); }
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
struct Rng {
    uint64_t st, inc;
    uint32_t key0, key1, t, env, dom, k;
    uint32_t blk;
    unsigned __int128 buf;   // the current Philox block, word j at bits 32j (no indexed fields)
    int mode;

    __device__ __forceinline__ void philox_block(uint32_t b) {
        uint32_t c0 = b, c1 = t, c2 = env, c3 = dom, k0 = key0, k1 = key1;
#pragma unroll
        for (int r = 0; r < 10; r++) {
            uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
            uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
            uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
            c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
            k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
        }
        buf = (unsigned __int128)c0 | ((unsigned __int128)c1 << 32) | ((unsigned __int128)c2 << 64) |
              ((unsigned __int128)c3 << 96);
        blk = b;
    }
    __device__ __forceinline__ uint32_t next() {
        if (mode == 0) {
            uint64_t old = st;
            st = old * 6364136223846793005ULL + (inc | 1);
            uint32_t x = (uint32_t)(((old >> 18) ^ old) >> 27), r = (uint32_t)(old >> 59);
            return (x >> r) | (x << ((0u - r) & 31u));
        }
        uint32_t b = k >> 2;
        if (b != blk) philox_block(b);
        uint32_t j = k & 3u;
        k++;
        return (uint32_t)(buf >> (32 * j));
    }
    __device__ __forceinline__ int r(int bound) {   // gpu-d1/src/sim.h:36-51
        if (bound <= 1) return 0;
        uint32_t x = next();
        uint64_t m = (uint64_t)x * (uint32_t)bound;
        uint32_t low = (uint32_t)m;
        if (low < (uint32_t)bound) {
            uint32_t th = (0u - (uint32_t)bound) % (uint32_t)bound;
            while (low < th) {
                x = next();
                m = (uint64_t)x * (uint32_t)bound;
                low = (uint32_t)m;
            }
        }
        return (int)(m >> 32);
    }
    __device__ __forceinline__ int avg(int n) { int a = r(n); return (a + r(n + 1)) / 2; }             // sim.h:52-55
    __device__ __forceinline__ int round(int n, int d) { int rem = n % d; return n / d + (rem && r(d) < rem); }  // sim.h:56-59
    __device__ __forceinline__ void pcg_seed(uint64_t s, uint64_t seq) {   // sim.h:29-35
        mode = 0; st = 0; inc = (seq << 1) | 1;
        next();
        st += s;
        next();
    }
    __device__ __forceinline__ void counter(uint64_t key, uint32_t e, uint32_t tt, uint32_t d) {
        mode = 1; key0 = (uint32_t)key; key1 = (uint32_t)(key >> 32); env = e; t = tt; dom = d; k = 0; blk = 0xFFFFFFFFu;
        st = 0; inc = 0;
    }
};

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
// Reservoir choice over `total` eligible cells: the 1-based count c is kept when
// r(c) == 0, the last kept count wins (gpu-d1/branches/d1-stairs-v2/src/learn.cu:432-441).
// 64 counts per pass: lane l evaluates count c0+l from the draw it would get if no
// earlier draw in the pass were rejected; a pass in which any Lemire rejection is
// possible (low < bound) is replayed serially, so the draw sequence is the serial one.
__device__ __forceinline__ int reservoir(Rng &s, int total, int lane) {
    int chosen = total >= 1 ? 0 : -1;
    int c0 = 2;
    while (c0 <= total) {
        int cnt = imin(64, total - c0 + 1);
        int c = c0 + lane;
        uint32_t xw;
        if (s.mode == 0) {
            uint64_t old = kJump.a[lane] * s.st + kJump.c[lane] * s.inc;
            xw = pcg_out(old);
        } else {
            uint32_t kk = s.k + (uint32_t)lane;
            Rng tmp = s;
            tmp.philox_block(kk >> 2);
            xw = (uint32_t)(tmp.buf >> (32 * (kk & 3u)));
        }
        uint64_t m = (uint64_t)xw * (uint32_t)c;
        bool act = lane < cnt;
        bool risky = act && (uint32_t)m < (uint32_t)c;
        if (ballot(risky)) {
            for (int cc = c0; cc < c0 + cnt; cc++) if (s.r(cc) == 0) chosen = cc - 1;
        } else {
            uint64_t keep = ballot(act && (m >> 32) == 0);
            if (keep) chosen = c0 + 63 - __clzll((long long)keep) - 1;
            if (s.mode == 0) s.st = kJump.a[cnt] * s.st + kJump.c[cnt] * s.inc;
            else s.k += (uint32_t)cnt;
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
    uint64_t vis0, vis1, vis2, vis3;   // player view, quadrants (+,+) (-,+) (-,-) (+,-)
    bool adj_clear;                     // the 8 neighbours of any cell are always in view
    // this lane's monster (lane < count)
    int mpos, mhp, menergy, mawake, mkind;
    int lane;
};

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
    if (dx >= 0 && dy >= 0) v |= x.vis0;
    if (dx <= 0 && dy >= 0) v |= x.vis1;
    if (dx <= 0 && dy <= 0) v |= x.vis2;
    if (dx >= 0 && dy <= 0) v |= x.vis3;
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
__device__ __forceinline__ void compute_view(Ctx &x) {
    int px = x.player % W, py = x.player / W;
    uint64_t o0 = opaque_set(x, px, py, 0), o1 = opaque_set(x, px, py, 1);
    uint64_t o2 = opaque_set(x, px, py, 2), o3 = opaque_set(x, px, py, 3);
    bool a0 = false, a1 = false, a2 = false, a3 = false;
    for (int s = 0; s < x.nslots; s++) {
        uint64_t m = x.rays[s * 64 + x.lane];
        a0 |= (m & o0) == 0; a1 |= (m & o1) == 0; a2 |= (m & o2) == 0; a3 |= (m & o3) == 0;
    }
    int tx = x.lane & 7, ty = x.lane >> 3;
    x.vis0 = ballot(a0 && inb(px + tx, py + ty));
    x.vis1 = ballot(a1 && inb(px - tx, py + ty));
    x.vis2 = ballot(a2 && inb(px - tx, py - ty));
    x.vis3 = ballot(a3 && inb(px + tx, py - ty));
}
// LOS from a monster to the player within Chebyshev 6 (monster_detects_player,
// gpu-d1/branches/d1-stairs-v2/src/learn.cu:199-207).
__device__ __forceinline__ bool detects(Ctx &x, int origin) {
    int ox = origin % W, oy = origin / W, dx = x.player % W - ox, dy = x.player / W - oy;
    if (iabs(dx) > 6 || iabs(dy) > 6) return false;
    if (!x.c->wake_los) return true;
    int t = iabs(dy) * 8 + iabs(dx);
    bool det = false;
    for (int q = 0; q < 4; q++) {
        bool sx = q_sx(q), sy = q_sy(q);
        if ((dx && (dx > 0) != sx) || (dy && (dy > 0) != sy)) continue;
        uint64_t opq = opaque_set(x, ox, oy, q);
        bool alive = x.lane < x.nslots && (x.rays[imin(x.lane, x.nslots - 1) * 64 + t] & opq) == 0;
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
        if (dy >= 0) { R |= (uint32_t)(x.vis0 >> (8 * ay)) & 0xFFu; L |= (uint32_t)(x.vis1 >> (8 * ay)) & 0xFFu; }
        if (dy <= 0) { R |= (uint32_t)(x.vis3 >> (8 * ay)) & 0xFFu; L |= (uint32_t)(x.vis2 >> (8 * ay)) & 0xFFu; }
        uint32_t v15 = (__builtin_bitreverse32(L) >> 24) | (R << 7);
        mask = row_place15(v15, px);
        Row old = row_ld(x.sm->viewed, y);
        Row fl = row_ld(x.sm->floor, y);
        fresh = row_popc(row_and(row_andn(mask, old), fl));
    }
    __syncthreads();
    if (mine) row_st(x.sm->viewed, y, row_or(mask, row_ld(x.sm->viewed, y)));
    __syncthreads();
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

// ---------------------------------------------------------------- episode reset
// gpu-d1/branches/d1-stairs-v2/src/learn.cu:351-446 (player, then monsters by
// rejection with the v1 HP table gpu-d1/src/learn.cu:305-314, then three stairs by
// reservoir choice from a copy of the RNG, then the initial reveal without reward).
// roster_mode 1 and awake_pct draw after the energy draw.
__device__ __forceinline__ void reset(Ctx &x, const uint32_t *cells_g) {
    Smem *sm = x.sm;
    const D1Config *c = x.c;
    for (int w = x.lane; w < ROWS_WORDS; w += 64) { sm->occ[w] = 0; sm->front[w] = cells_g[w]; sm->viewed[w] = 0; }
    __syncthreads();
    x.ncells = row_prefix(x, sm->front);
    x.player = select_cell(x, sm->front, x.g.r(x.ncells));
    x.hp = c->hp; x.regen = 0; x.blocks = 0;
    x.ticks = 0; x.decisions = 0; x.killed = 0; x.floor_seen = 0;
    int mpos = -1, mhp = 0, men = -30000, mawake = 0, mkind = 0;
    for (int i = 0; i < c->count; i++) {
        int p = 0, tries = 0;
        do {
            p = select_cell(x, sm->front, x.g.r(x.ncells));
            tries++;
        } while ((p == x.player || bit(sm->occ, p)) && tries < 65536);
        if (p == x.player || bit(sm->occ, p)) {   // unreachable in practice; first free cell
            for (int j = 0; j < x.ncells; j++) {
                p = select_cell(x, sm->front, j);
                if (p != x.player && !bit(sm->occ, p)) break;
            }
        }
        occ_set(x, p, true);
        int kind = i % 6, hpv = 0;
        if (c->roster_mode == 0) { const int MHP[6] = {8, 10, 12, 16, 12, 10}; hpv = MHP[i % 6]; }
        int en = 70 + x.g.r(10);
        if (c->roster_mode == 1) { kind = x.g.r(6); hpv = c->hp_lo + x.g.r(c->hp_hi - c->hp_lo + 1); }
        int aw = c->awake_pct >= 100 ? 1 : c->awake_pct <= 0 ? 0 : (x.g.r(100) < c->awake_pct);
        if (x.lane == i) { mpos = p; mhp = hpv; men = en; mawake = aw; mkind = kind; }
    }
    x.mpos = mpos; x.mhp = mhp; x.menergy = men; x.mawake = mawake; x.mkind = mkind;
    // Stairs: a copy of the RNG, reservoir over eligible cells in cell order.
    Rng s = x.g;
    x.first_stair_tick = -1;
    x.stairs = pack_stairs(-1, -1, -1);
    int px = x.player % W, py = x.player / W;
    for (int k = 0; k < 3; k++) {
        if (k >= c->stairs) break;
        // eligible rows into sm->reach: cells & ~occ & cheb(player) >= 12 & cheb(prev stairs) >= 8
        for (int y = x.lane; y < H; y += 64) {
            Row e = row_andn(row_ld(sm->front, y), row_ld(sm->occ, y));
            if (iabs(y - py) < 12) e = row_andn(e, row_range(px - 11, px + 11));
            for (int q = 0; q < k; q++) {
                int sp = stair_at(x, q);
                if (iabs(y - sp / W) < 8) e = row_andn(e, row_range(sp % W - 7, sp % W + 7));
            }
            row_st(sm->reach, y, e);
        }
        __syncthreads();
        int total = row_prefix(x, sm->reach);
        int chosen = reservoir(s, total, x.lane);
        int sel = chosen >= 0 ? select_cell(x, sm->reach, chosen) : -1;
        x.stairs = (x.stairs & ~(0xFFFFULL << (16 * k))) | (uint64_t)(uint16_t)sel << (16 * k);
        __syncthreads();
    }
    reveal(x);
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
    const D1Kind &k = c->kinds[kind];
    Rng &r = x.g;
    int hit = r.r(k.tohit + 1);
    int ev = r.round(c->ev100, 100);
    ev = r.avg(2 * ev);
    int margin = hit - ev;
    if (r.r(100) < 5) margin = (r.r(2) ? 1 : -1) * 1000;
    int bypass = r.r(k.bypass);
    int sh = r.round(c->sh100, 100);
    int block = r.avg(sh * 2) / 3 - 1;
    if (block >= bypass && x.blocks < c->shield_limit) { x.blocks++; return; }
    if (margin < 0) return;
    int damage = 1 + r.r(k.damage);
    int ac = r.round(c->ac100, 100);
    int gac = r.round(c->ac100, 100);
    int gdr = c->gdr[imin(imax(gac - c->ac100 / 100, 0), 1)];
    int saved = r.r(ac + 1);
    int half = r.round(ac, 2);
    saved = imax(saved, imin(gdr * k.damage / 100, half));
    damage = imax(0, damage - saved);
    x.hp -= damage;
}
// distance of q relative to p (both via the BFS field); BIG when q was not reached
__device__ __forceinline__ int rel_dist(const Ctx &x, int q, int p) {
    if (!bit(x.sm->reach, q)) return BIG;
    return (int)(int8_t)(uint8_t)(x.sm->dist[q] - x.sm->dist[p]);
}
__device__ __forceinline__ bool walkable(const Ctx &x, int q) {
    return q >= 0 && bit(x.sm->floor, q) && q != x.player && !bit(x.sm->occ, q);
}
// gpu-d1/src/sim.h:207-253: greedy descent with rotated order and 1/ties
// replacement, then a bounded 24-node BFS detour when stuck.
__device__ __forceinline__ int choose_move(Ctx &x, int p) {
    int rotation = x.g.r(4);
    int z = x.lane & 7;
    int d = z < 4 ? (z + rotation) % 4 : 4 + (z + rotation) % 4;
    int q = nbr(p, d);
    bool ok = x.lane < 8 && walkable(x, q);
    int rel = ok ? rel_dist(x, q, p) : BIG;
    uint64_t okm = ballot(ok);
    int best = -1, bd = 0, ties = 0;
    for (int zz = 0; zz < 8; zz++) {
        if (!((okm >> zz) & 1)) continue;
        int dd = lane_val(rel, zz), qq = lane_val(q, zz);
        if (dd < bd) { bd = dd; best = qq; ties = 1; }
        else if (dd == bd && best >= 0 && x.g.r(++ties) == 0) best = qq;
    }
    if (best >= 0 || !x.c->repair) return best;
    // queue: lane j holds cells[j] and first[j]
    int qcell = x.lane == 0 ? p : -1, qfirst = -1, len = 1;
    for (int head = 0; head < len; head++) {
        int cell = lane_val(qcell, head);
        int hfirst = lane_val(qfirst, head);
        int nq = nbr(cell, x.lane & 7);
        bool v = x.lane < 8 && walkable(x, nq);
        uint64_t vm = ballot(v);
        for (int dd = 0; dd < 8; dd++) {
            if (!((vm >> dd) & 1)) continue;
            int qq = lane_val(nq, dd);
            if (ballot(x.lane < len && qcell == qq)) continue;
            int step = head == 0 ? qq : hfirst;
            if (rel_dist(x, qq, p) < 0) return step;
            if (len < 24) {
                if (x.lane == len) { qcell = qq; qfirst = step; }
                len++;
            }
        }
    }
    return -1;
}
// One BFS layer for row y: dilate the frontier rows y-1..y+1 by one cell, keep floor
// cells not reached yet.
__device__ __forceinline__ Row bfs_expand(const Smem *sm, int y) {
    Row v = row_ld(sm->front, y);
    if (y > 0) v = row_or(v, row_ld(sm->front, y - 1));
    if (y < H - 1) v = row_or(v, row_ld(sm->front, y + 1));
    v = row_or(v, row_or(row_shl1(v), row_shr1(v)));
    return row_andn(row_and(v, row_ld(sm->floor, y)), row_ld(sm->reach, y));
}
__device__ __forceinline__ void scatter_layer(Smem *sm, int base, uint32_t b, int layer) {
    while (b) {
        int xx = __ffs(b) - 1;
        b &= b - 1;
        sm->dist[base + xx] = (uint8_t)layer;
    }
}
__device__ __forceinline__ void bfs_commit(Smem *sm, int y, Row nw, int layer) {
    row_st(sm->front, y, nw);
    row_st(sm->reach, y, row_or(row_ld(sm->reach, y), nw));
    scatter_layer(sm, y * W, nw.a, layer);
    scatter_layer(sm, y * W + 32, nw.b, layer);
    scatter_layer(sm, y * W + 64, nw.c, layer);
}
// Bit-parallel BFS over floor from the player (the all-pairs row of
// gpu-d1/scripts/learn_env.py:31-39), stopped `margin` layers after every mover is
// reached. dist holds the layer mod 256; comparisons are relative (|delta| <= 25).
__device__ __forceinline__ void bfs(Ctx &x, uint64_t movers, int margin) {
    Smem *sm = x.sm;
    for (int w = x.lane; w < ROWS_WORDS; w += 64) { sm->reach[w] = 0; sm->front[w] = 0; }
    __syncthreads();
    if (x.lane == 0) {
        int p = x.player;
        sm->reach[(p / W) * RW + ((p % W) >> 5)] |= 1u << ((p % W) & 31);
        sm->front[(p / W) * RW + ((p % W) >> 5)] |= 1u << ((p % W) & 31);
        sm->dist[p] = 0;
    }
    __syncthreads();
    int stop = 1 << 30;
    const int y0 = x.lane, y1 = x.lane + 64;
    for (int layer = 1; layer < N; layer++) {
        Row n0 = bfs_expand(sm, y0), n1 = y1 < H ? bfs_expand(sm, y1) : Row{0, 0, 0};
        __syncthreads();
        bfs_commit(sm, y0, n0, layer);
        if (y1 < H) bfs_commit(sm, y1, n1, layer);
        __syncthreads();
        if (!ballot(row_any(n0) || row_any(n1))) break;
        if (stop == (1 << 30)) {
            bool missing = ((movers >> x.lane) & 1) && !bit(sm->reach, x.mpos);
            if (!ballot(missing)) stop = layer + margin;
        }
        if (layer >= stop) break;
    }
}
// gpu-d1/src/sim.h:254-269
__device__ __forceinline__ void act(Ctx &x, int id) {
    if (x.lane == id) x.menergy -= 10;
    int p = lane_val(x.mpos, id);
    if (cheb(p, x.player) == 1) { attack(x, lane_val(x.mkind, id)); return; }
    int q = choose_move(x, p);
    if (q >= 0) {
        occ_set(x, p, false);
        occ_set(x, q, true);
        if (x.lane == id) x.mpos = q;
    }
}

// ---------------------------------------------------------------- one physical turn
// gpu-d1/branches/d1-stairs-v2/src/learn.cu:684-827 with the v1 kill-all clear
// (gpu-d1/src/learn.cu:549) as a switch. d: 0-7 move/bump, 8 wait, 18 descend.
// Returns done; out8 = reward, done, clear, killed, hp, ticks, death, timeout.
__device__ __forceinline__ bool primitive(Ctx &x, int d, float *out8, bool &saw, const uint32_t *cells_g) {
    const D1Config *c = x.c;
    Smem *sm = x.sm;
    int milli = c->step_milli;
    x.blocks = 0;
    x.regen += c->regen;
    while (x.regen >= 100) { x.hp = imin(c->hp, x.hp + 1); x.regen -= 100; }
    if (d >= 0 && d < 8) {
        int p = nbr(x.player, d);
        if (p >= 0 && bit(sm->floor, p)) {
            uint64_t at = ballot(x.lane < c->count && x.mhp > 0 && x.mpos == p);
            if (at) {
                int id = __ffsll((unsigned long long)at) - 1;
                if (x.g.r(5) != 0) {
                    int dmg = 1 + x.g.r(4);
                    int nh = (int16_t)(lane_val(x.mhp, id) - dmg);
                    if (nh <= 0) {
                        if (x.lane == id) { x.mhp = 0; x.menergy = -30000; }
                        occ_set(x, p, false);
                        x.killed++;
                        milli += c->kill_milli;
                    } else if (x.lane == id) x.mhp = nh;
                }
            } else x.player = p;
        }
    }
    milli += c->explore_milli * reveal(x);
    saw = visible_awake(x);
    bool clear = (d == 18 && stair_index(x) > 0 && x.hp > 0) || (c->clear_on_kill_all && x.killed == c->count);
    if (!clear) {
        bool mine = x.lane < c->count;
        uint64_t cand = ballot(mine && x.mhp > 0 && !x.mawake && cheb(x.mpos, x.player) <= 6);
        while (cand) {
            int i = __ffsll((unsigned long long)cand) - 1;
            cand &= cand - 1;
            int pos = lane_val(x.mpos, i);
            if (detects(x, pos) && x.lane == i) { x.mawake = 1; x.menergy = 70; }
        }
        if (mine && x.mhp > 0 && !x.mawake) x.menergy = -30000;
        int maxspeed = 0;
        if (mine && x.mhp > 0) x.menergy += kind_speed(c, x.mkind);
        for (int k = 0; k < 6; k++) maxspeed = imax(maxspeed, c->kinds[k].speed);
        x.menergy = (int16_t)x.menergy;
        uint64_t movers = ballot(mine && x.mhp > 0 && x.mawake && x.menergy >= 80 && cheb(x.mpos, x.player) > 1);
        if (movers) bfs(x, movers, imax(2, (maxspeed + 9) / 10));
        while (x.hp > 0) {
            int key = (mine && x.menergy >= 80) ? x.menergy * 128 + 127 - x.lane : -1;
            key = wave_max(key);
            if (key < 0) break;
            int id = 127 - (key & 127);
            act(x, id);
            if (in_view(x, lane_val(x.mpos, id))) saw = true;
        }
    }
    x.ticks++;
    if (x.first_stair_tick < 0 && known_stairs(x) > 0) x.first_stair_tick = x.ticks;
    bool death = x.hp <= 0, timeout = !clear && !death && x.ticks >= c->limit;
    if (clear) milli += c->clear_milli;
    if (death) milli -= c->death_milli;
    float reward = 0.001f * (float)milli;
    reward -= c->turn_cost;
    saw = saw || visible_awake(x);
    bool done = clear || death || timeout;
    out8[0] = reward; out8[1] = done; out8[2] = clear; out8[3] = (float)x.killed;
    out8[4] = (float)imax(0, x.hp); out8[5] = (float)x.ticks; out8[6] = death; out8[7] = timeout;
    if (done) { x.episode++; reset(x, cells_g); }
    return done;
}

// Joint action, gpu-d1/branches/d1-stairs-v2/src/learn.cu:852-875.
__device__ __forceinline__ void transition(Ctx &x, int action, float *out, const uint32_t *cells_g) {
    const D1Config *c = x.c;
    int decisions = x.decisions + 1;
    bool invalid = false;
    float total = 0.f, out8[8];
    for (int guard = 0; guard < 1 << 16; guard++) {
        int d = 8;
        if (action >= 0 && action < 16) {
            int dir = action % 8, p = nbr(x.player, dir);
            bool enemy = p >= 0 && (x.adj_clear || in_view(x, p)) && bit(x.sm->occ, p);
            bool valid = action < 8 ? p >= 0 && (!bit(x.sm->viewed, p) || bit(x.sm->floor, p)) && !enemy : enemy;
            if (valid) d = dir; else invalid = true;
        } else if (action == 17) invalid = x.hp >= c->hp || visible_awake(x) || c->regen <= 0;
        else if (action == 18) { if (stair_index(x) > 0) d = 18; else invalid = true; }
        else if (action != 16) invalid = true;
        bool saw = false;
        bool done = primitive(x, d, out8, saw, cells_g);
        total += out8[0];
        if (done || invalid || action != 17) break;
        if (saw || x.hp >= c->hp) break;
    }
    out[0] = total;
    for (int j = 1; j < 8; j++) out[j] = out8[j];
    if (out8[1] == 0.f) x.decisions = decisions;
}

// ---------------------------------------------------------------- observation + hash
// uint8 [15][15][8]: 0 wall (out of bounds or viewed non-floor), 1 viewed floor,
// 2 visible, 3 monster kind+1, 4 monster HP (visible, living), 5 player HP,
// 6 remembered stair, 7 frontier anchor (seen floor with an in-bounds unviewed
// neighbour; the FRONTIER_RING_MEMORY_WALLS rule of
// gpu-d1/branches/d1-stairs-v2/src/learn.cu:269-280).
__device__ __forceinline__ void write_obs(Ctx &x, uint8_t *o) {
    Smem *sm = x.sm;
    int px = x.player % W, py = x.player / W;
    // frontier rows of the window into sm->front
    {
        int y = py + x.lane - 7;
        if (x.lane < 15 && y >= 0 && y < H) {
            const Row all = row_range(0, W - 1);
            Row u{0, 0, 0};
            for (int yy = y - 1; yy <= y + 1; yy++)
                if (yy >= 0 && yy < H) u = row_or(u, row_andn(all, row_ld(sm->viewed, yy)));
            u = row_and(row_or(u, row_or(row_shl1(u), row_shr1(u))), all);
            Row f = row_and(row_and(row_ld(sm->floor, y), row_ld(sm->viewed, y)), u);
            row_st(sm->front, y, f);
        }
    }
    for (int cidx = x.lane; cidx < 225; cidx += 64) sm->win[cidx] = 0;
    __syncthreads();
    if (x.lane < x.c->count && x.mhp > 0) {
        int dx = x.mpos % W - px, dy = x.mpos / W - py;
        if (iabs(dx) <= 7 && iabs(dy) <= 7)
            sm->win[(dy + 7) * 15 + dx + 7] = (uint32_t)(x.mkind + 1) | ((uint32_t)imin(x.mhp, 255) << 8);
    }
    __syncthreads();
    for (int k = 0; k < 3; k++) {
        int sp = stair_at(x, k);
        if (x.lane == 0 && sp >= 0) {
            int dx = sp % W - px, dy = sp / W - py;
            if (iabs(dx) <= 7 && iabs(dy) <= 7) sm->win[(dy + 7) * 15 + dx + 7] |= 1u << 16;
        }
    }
    __syncthreads();
    uint32_t php = (uint32_t)imin(imax(x.hp, 0), 255);
    for (int cidx = x.lane; cidx < 225; cidx += 64) {
        int dy = cidx / 15 - 7, dx = cidx % 15 - 7, xx = px + dx, yy = py + dy;
        uint32_t lo = 0, hi = php << 8;   // bytes 4..7 = ch4 hp, ch5 player hp, ch6 stair, ch7 frontier
        if (!inb(xx, yy)) lo = 1;
        else {
            bool vw = bit_at(sm->viewed, xx, yy), fl = bit_at(sm->floor, xx, yy);
            bool vis = vis_rel(x, dx, dy);
            uint32_t wv = sm->win[cidx];
            lo = (uint32_t)(vw && !fl) | ((uint32_t)(vw && fl) << 8) | ((uint32_t)vis << 16);
            if (vis && (wv & 0xFFu)) { lo |= (wv & 0xFFu) << 24; hi |= (wv >> 8) & 0xFFu; }
            if ((wv >> 16) & 1u && vw && fl) hi |= 1u << 16;
            if (bit_at(sm->front, xx, yy)) hi |= 1u << 24;
        }
        *(uint2 *)(o + cidx * 8) = make_uint2(lo, hi);
    }
}
// Sum over canonical words of fmix32(word ^ index*0x9E3779B9) (index map in
// include/d1hip.h's companion spec: scalars 0-14, monsters 100+2i, viewed 1000+3y+j).
__device__ __forceinline__ uint32_t state_hash(Ctx &x) {
    // scalar words are hashed in uniform code and added once (lane 0)
    uint32_t scal = term((uint32_t)x.player, 0) + term((uint32_t)x.hp, 1) + term((uint32_t)x.regen, 2) +
                    term((uint32_t)x.ticks, 3) + term((uint32_t)x.killed, 4) + term((uint32_t)x.decisions, 5) +
                    term((uint32_t)x.floor_seen, 6) + term((uint32_t)x.episode, 7) +
                    term(x.g.mode == 0 ? (uint32_t)x.g.st : 0u, 8) + term(x.g.mode == 0 ? (uint32_t)(x.g.st >> 32) : 0u, 9) +
                    term(x.t, 10) + term((uint32_t)stair_at(x, 0), 11) + term((uint32_t)stair_at(x, 1), 12) +
                    term((uint32_t)stair_at(x, 2), 13) + term((uint32_t)x.first_stair_tick, 14);
    uint32_t h = x.lane == 0 ? scal : 0u;
    if (x.lane < x.c->count) {
        h += term((uint16_t)x.mpos | (uint32_t)(uint16_t)x.mhp << 16, 100 + 2 * x.lane);
        h += term((uint16_t)x.menergy | (uint32_t)x.mawake << 16 | (uint32_t)x.mkind << 24, 101 + 2 * x.lane);
    }
    for (int y = x.lane; y < H; y += 64)
        for (int j = 0; j < 3; j++) h += term(x.sm->viewed[y * RW + j], 1000 + 3 * y + j);
    return wave_sum(h);
}

// ---------------------------------------------------------------- load / store
__device__ __forceinline__ void load_world(Ctx &x, const uint8_t *row, int max_m) {
    Hdr h = *(const Hdr *)row;
    x.player = h.player; x.hp = h.hp; x.regen = h.regen; x.ncells = h.ncells;
    x.ticks = h.ticks; x.killed = h.killed; x.decisions = h.decisions; x.floor_seen = h.floor_seen;
    x.episode = h.episode; x.first_stair_tick = h.first_stair_tick;
    x.stairs = pack_stairs(h.stairs[0], h.stairs[1], h.stairs[2]);
    x.blocks = h.blocks; x.t = h.t; x.env_id = h.env_id;
    if (x.c->rng_mode == 0) { x.g.mode = 0; x.g.st = h.rng_state; x.g.inc = h.rng_inc; }
    else x.g.counter(h.rng_state, h.env_id, h.t, 0);
    Mon m{-1, 0, -30000, 0, 0};
    if (x.lane < max_m) m = ((const Mon *)(row + 64))[x.lane];
    x.mpos = m.pos; x.mhp = m.hp; x.menergy = m.energy; x.mawake = m.awake; x.mkind = m.kind;
    const uint32_t *vg = (const uint32_t *)(row + off_viewed(max_m));
    const uint32_t *fg = (const uint32_t *)(row + off_floor(max_m));
    for (int w = x.lane; w < ROWS_WORDS; w += 64) { x.sm->viewed[w] = vg[w]; x.sm->floor[w] = fg[w]; x.sm->occ[w] = 0; }
    __syncthreads();
    if (x.lane < x.c->count && x.mhp > 0)
        atomicOr(&x.sm->occ[(x.mpos / W) * RW + ((x.mpos % W) >> 5)], 1u << ((x.mpos % W) & 31));
    __syncthreads();
}
__device__ __forceinline__ void store_world(Ctx &x, uint8_t *row, int max_m) {
    if (x.lane == 0) {
        Hdr h;
        h.rng_state = x.g.mode == 0 ? x.g.st : ((uint64_t)x.g.key1 << 32 | x.g.key0);
        h.rng_inc = x.g.mode == 0 ? x.g.inc : 0;
        h.env_id = x.env_id; h.t = x.t; h.episode = x.episode;
        h.player = (int16_t)x.player; h.hp = (int16_t)x.hp; h.regen = (int16_t)x.regen; h.ncells = (int16_t)x.ncells;
        h.ticks = x.ticks; h.killed = x.killed; h.decisions = x.decisions; h.floor_seen = x.floor_seen;
        h.stairs[0] = (int16_t)stair_at(x, 0); h.stairs[1] = (int16_t)stair_at(x, 1); h.stairs[2] = (int16_t)stair_at(x, 2);
        h.blocks = (int16_t)x.blocks; h.first_stair_tick = x.first_stair_tick;
        *(Hdr *)row = h;
    }
    if (x.lane < x.c->count) {
        Mon m;
        m.pos = (int16_t)x.mpos; m.hp = (int16_t)x.mhp; m.energy = (int16_t)x.menergy;
        m.awake = (uint8_t)x.mawake; m.kind = (uint8_t)x.mkind;
        ((Mon *)(row + 64))[x.lane] = m;
    }
    uint32_t *vg = (uint32_t *)(row + off_viewed(max_m));
    for (int w = x.lane; w < ROWS_WORDS; w += 64) vg[w] = x.sm->viewed[w];
}

// ---------------------------------------------------------------- level generator
// Build-owned spec (see oracle/d1_oracle.c o_level_generate): 3x3 sectors, 6-9
// rooms by partial Fisher-Yates, L corridors between consecutive centres.
__device__ __forceinline__ void generate_level(Ctx &x, uint64_t seed, uint32_t env, uint32_t *floor_rows) {
    Rng g;
    g.counter(seed, env, 0, 1);
    int n = 6 + g.r(4);
    uint64_t order = 0x876543210ULL;   // nibble i = sector at position i
    for (int i = 0; i < n; i++) {
        int j = i + g.r(9 - i);
        uint64_t a = (order >> (4 * i)) & 15, b = (order >> (4 * j)) & 15;
        order &= ~((15ULL << (4 * i)) | (15ULL << (4 * j)));
        order |= (b << (4 * i)) | (a << (4 * j));
    }
    int rx = 0, ry = 0, rw = 0, rh = 0, vf = 0;   // lane i holds room i and corridor i-1 -> i
    for (int i = 0; i < n; i++) {
        int s = (int)((order >> (4 * i)) & 15);
        int x0 = 1 + 26 * (s % 3), y0 = 1 + 22 * (s / 3);
        int w = 4 + g.r(9), h = 3 + g.r(6);
        int xx = x0 + g.r(27 - w), yy = y0 + g.r(23 - h);
        if (x.lane == i) { rx = xx; ry = yy; rw = w; rh = h; }
    }
    for (int i = 1; i < n; i++) {
        int v = g.r(2);
        if (x.lane == i) vf = v;
    }
    for (int s = 0; s < 2; s++) {
        int y = x.lane + 64 * s;
        if (s == 1 && y >= H) break;
        Row r{0, 0, 0};
        for (int i = 0; i < n; i++) {
            int ax = lane_val(rx, i), ay = lane_val(ry, i), aw = lane_val(rw, i), ah = lane_val(rh, i);
            if (y >= ay && y < ay + ah) r = row_or(r, row_range(ax, ax + aw - 1));
            if (i > 0) {
                int bx = lane_val(rx, i - 1) + lane_val(rw, i - 1) / 2, by = lane_val(ry, i - 1) + lane_val(rh, i - 1) / 2;
                int cx2 = ax + aw / 2, cy2 = ay + ah / 2, v = lane_val(vf, i);
                int hy = v ? cy2 : by, vx = v ? bx : cx2;
                if (y == hy) r = row_or(r, row_range(imin(bx, cx2), imax(bx, cx2)));
                if (y >= imin(by, cy2) && y <= imax(by, cy2)) r = row_or(r, row_range(vx, vx));
            }
        }
        if (y < H) row_st(floor_rows, y, r);
    }
}

// ---------------------------------------------------------------- kernels
__global__ __launch_bounds__(64) void k_init(uint8_t *state, int n, int max_m, size_t row_bytes, D1Config cfg,
                                             D1Tables tab, uint64_t seed, uint8_t *obs, uint32_t *hash) {
    __shared__ Smem sm;
    int env = blockIdx.x;
    if (env >= n) return;
    uint8_t *row = state + (size_t)env * row_bytes;
    Ctx x;
    x.sm = &sm; x.c = &cfg; x.rays = tab.ray_slots; x.nslots = tab.nslots; x.lane = lane_id();
    x.adj_clear = false;
    uint32_t *fg = (uint32_t *)(row + off_floor(max_m));
    uint32_t *cg = (uint32_t *)(row + off_cells(max_m));
    if (cfg.level_mode == 1) {
        generate_level(x, seed, (uint32_t)env, sm.floor);
        __syncthreads();
        for (int w = x.lane; w < ROWS_WORDS; w += 64) { fg[w] = sm.floor[w]; cg[w] = sm.floor[w]; }
    } else {
        for (int s = 0; s < 2; s++) {
            int y = x.lane + 64 * s;
            if (y >= H) break;
            for (int j = 0; j < 3; j++) {
                uint32_t f = 0, cc = 0;
                for (int b = 0; b < 32 && 32 * j + b < W; b++) {
                    f |= (uint32_t)(tab.floor[y * W + 32 * j + b] != 0) << b;
                    cc |= (uint32_t)(tab.cells[y * W + 32 * j + b] != 0) << b;
                }
                sm.floor[y * RW + j] = f; fg[y * RW + j] = f; cg[y * RW + j] = cc;
            }
        }
    }
    __syncthreads();
    __threadfence_block();
    x.env_id = (uint32_t)env; x.t = 0; x.episode = 0;
    if (cfg.rng_mode == 0) x.g.pcg_seed(mix64(seed + (uint64_t)env), (uint64_t)env + 1);
    else x.g.counter(seed, (uint32_t)env, 0, 2);
    x.decisions = 0; x.floor_seen = 0;
    reset(x, cg);
    store_world(x, row, max_m);
    if (obs) write_obs(x, obs + (size_t)env * D1_OBS_BYTES);
    uint32_t h = state_hash(x);
    if (hash && x.lane == 0) hash[env] = h;
}

__global__ __launch_bounds__(64) void k_step(uint8_t *state, int n, int max_m, size_t row_bytes, D1Config cfg,
                                             D1Tables tab, const int64_t *actions, uint8_t *obs, float *out,
                                             uint32_t *hash, const uint8_t *active) {
    __shared__ Smem sm;
    int env = blockIdx.x;
    if (env >= n) return;
    if (active && !active[env]) return;
    uint8_t *row = state + (size_t)env * row_bytes;
    Ctx x;
    x.sm = &sm; x.c = &cfg; x.rays = tab.ray_slots; x.nslots = tab.nslots; x.lane = lane_id();
    load_world(x, row, max_m);
    const uint32_t *cg = (const uint32_t *)(row + off_cells(max_m));
    int64_t a = actions[env];
    int action = a < 0 || a > 1000 ? -1 : (int)a;
    // Adjacent cells are visible whenever their first ray has no blocker (true of the
    // native table); then only REST needs the full view before the player acts.
    x.adj_clear = tab.ray_slots[1] == 0 && tab.ray_slots[8] == 0 && tab.ray_slots[9] == 0;
    if (!x.adj_clear || action == 17) compute_view(x);
    float o8[8];
    transition(x, action, o8, cg);
    x.t++;
    store_world(x, row, max_m);
    if (out && x.lane == 0) {
        float4 *o4 = (float4 *)(out + (size_t)env * D1_OUT);
        o4[0] = make_float4(o8[0], o8[1], o8[2], o8[3]);
        o4[1] = make_float4(o8[4], o8[5], o8[6], o8[7]);
    }
    if (obs) write_obs(x, obs + (size_t)env * D1_OBS_BYTES);
    uint32_t h = state_hash(x);
    if (hash && x.lane == 0) hash[env] = h;
}

// ---------------------------------------------------------------- monster-wait workload
// The reference's wait benchmark (gpu-d1/src/bench.cu:36-96,151-184 over
// gpu-d1/src/sim.h:93-122,276-295): a stationary player on a fixed map, `count` awake
// monsters at a fixture spawn list, a static distance-from-player field; one call runs
// `steps` waits per world. World row (WAIT_BYTES): header then {i16 pos, i16 energy} x 64.
constexpr int WAIT_BYTES = 64 + 4 * 64;
struct WaitHdr {
    uint64_t rng_state, rng_inc;
    int32_t hp, regen, blocks, fixture, episode;
    int32_t pad[7];
};
static_assert(sizeof(WaitHdr) == 64, "wait header");

__device__ __forceinline__ void wait_stage_map(Ctx &x, const D1WaitMap &map) {
    Smem *sm = x.sm;
    for (int s = 0; s < 2; s++) {
        int y = x.lane + 64 * s;
        if (y >= H) break;
        for (int j = 0; j < 3; j++) {
            uint32_t f = 0, r = 0;
            for (int b = 0; b < 32 && 32 * j + b < W; b++) {
                int p = y * W + 32 * j + b;
                f |= (uint32_t)(map.floor[p] != 0) << b;
                r |= (uint32_t)(map.dist[p] != 65535) << b;
            }
            sm->floor[y * RW + j] = f;
            sm->reach[y * RW + j] = r;
            sm->occ[y * RW + j] = 0;
        }
    }
    for (int p = x.lane; p < N; p += 64) sm->dist[p] = (uint8_t)map.dist[p];
    __syncthreads();
}
// gpu-d1/src/sim.h:93-111
__device__ __forceinline__ void wait_reset(Ctx &x, const D1WaitMap &map, int count, int fixture, bool first) {
    if (!first && x.lane < count) occ_clear_lane(x, x.mpos);
    __syncthreads();
    x.hp = x.c->hp; x.regen = 0; x.blocks = 0;
    for (int i = 0; i < count; i++) {
        int p = map.starts[fixture * 64 + i];
        int en = 70 + x.g.r(10);
        if (x.lane == i) { x.mpos = p; x.menergy = en; }
    }
    if (x.lane < count) occ_set_lane(x, x.mpos);
    __syncthreads();
    if (!first) x.episode++;
}
// gpu-d1/src/sim.h:112-122,276-295 (scan scheduler; the heap picks the same actors)
__device__ __forceinline__ void wait_step(Ctx &x, const D1WaitMap &map, int count, int fixture) {
    if (x.hp <= 0) wait_reset(x, map, count, fixture, false);
    x.blocks = 0;
    x.regen += x.c->regen;
    while (x.regen >= 100) { x.hp = imin(x.c->hp, x.hp + 1); x.regen -= 100; }
    bool mine = x.lane < count;
    if (mine) x.menergy = (int16_t)(x.menergy + kind_speed(x.c, x.mkind));
    while (x.hp > 0) {
        int key = (mine && x.menergy >= 80) ? x.menergy * 128 + 127 - x.lane : -1;
        key = wave_max(key);
        if (key < 0) break;
        act(x, 127 - (key & 127));
    }
}
__device__ __forceinline__ uint32_t wait_digest(Ctx &x, int count) {
    uint32_t h = x.lane < count ? term((uint16_t)x.mpos | (uint32_t)(uint16_t)x.menergy << 16, 100 + x.lane) : 0u;
    h = wave_sum(h);
    return h + term((uint32_t)x.hp, 0) + term((uint32_t)x.regen, 1) + term((uint32_t)x.blocks, 2) +
           term((uint32_t)x.episode, 3) + term((uint32_t)x.g.st, 4) + term((uint32_t)(x.g.st >> 32), 5);
}
__device__ __forceinline__ void wait_load(Ctx &x, const uint8_t *row, int count, int &fixture) {
    WaitHdr h = *(const WaitHdr *)row;
    x.g.mode = 0; x.g.st = h.rng_state; x.g.inc = h.rng_inc;
    x.hp = h.hp; x.regen = h.regen; x.blocks = h.blocks; x.episode = h.episode; fixture = h.fixture;
    x.mpos = -1; x.menergy = -30000; x.mkind = x.lane % 6; x.mhp = 1; x.mawake = 1;
    if (x.lane < count) {
        const int16_t *m = (const int16_t *)(row + 64) + 2 * x.lane;
        x.mpos = m[0]; x.menergy = m[1];
        occ_set_lane(x, x.mpos);
    }
    __syncthreads();
}
__device__ __forceinline__ void wait_store(Ctx &x, uint8_t *row, int count, int fixture) {
    if (x.lane == 0) {
        WaitHdr h{};
        h.rng_state = x.g.st; h.rng_inc = x.g.inc;
        h.hp = x.hp; h.regen = x.regen; h.blocks = x.blocks; h.fixture = fixture; h.episode = x.episode;
        *(WaitHdr *)row = h;
    }
    if (x.lane < count) {
        int16_t *m = (int16_t *)(row + 64) + 2 * x.lane;
        m[0] = (int16_t)x.mpos; m[1] = (int16_t)x.menergy;
    }
}
__device__ __forceinline__ void wait_ctx(Ctx &x, Smem *sm, const D1Config *cfg, const D1WaitMap &map) {
    x.sm = sm; x.c = cfg; x.rays = nullptr; x.nslots = 0; x.lane = lane_id(); x.adj_clear = true;
    x.player = map.player; x.vis0 = x.vis1 = x.vis2 = x.vis3 = 0;
}
// scenario 0 contact, 1 approach, 2 mixed (fixture = world % 2, then (world*7)%32 warm-up
// waits), as gpu-d1/src/bench.cu:151-166.
__global__ __launch_bounds__(64) void k_wait_init(uint8_t *worlds, int n, int count, D1Config cfg, D1WaitMap map,
                                                  uint64_t seed, int scenario) {
    __shared__ Smem sm;
    int w = blockIdx.x;
    if (w >= n) return;
    Ctx x;
    wait_ctx(x, &sm, &cfg, map);
    wait_stage_map(x, map);
    x.g.pcg_seed(mix64(seed + (uint64_t)w), (uint64_t)w + 1);
    int fixture = scenario == 1 ? 1 : scenario == 2 ? w % 2 : 0;
    x.episode = 0;
    x.mpos = -1; x.menergy = -30000; x.mkind = x.lane % 6; x.mhp = 1; x.mawake = 1;
    wait_reset(x, map, count, fixture, true);
    int warm = scenario == 2 ? (w * 7) % 32 : 0;
    for (int k = 0; k < warm; k++) wait_step(x, map, count, fixture);
    wait_store(x, worlds + (size_t)w * WAIT_BYTES, count, fixture);
}
__global__ __launch_bounds__(64) void k_wait(uint8_t *worlds, int n, int count, D1Config cfg, D1WaitMap map, int steps,
                                             uint32_t *trace) {
    __shared__ Smem sm;
    int w = blockIdx.x;
    if (w >= n) return;
    Ctx x;
    wait_ctx(x, &sm, &cfg, map);
    wait_stage_map(x, map);
    int fixture = 0;
    uint8_t *row = worlds + (size_t)w * WAIT_BYTES;
    wait_load(x, row, count, fixture);
    for (int k = 0; k < steps; k++) {
        wait_step(x, map, count, fixture);
        if (trace) {
            uint32_t h = wait_digest(x, count);
            if (x.lane == 0) trace[(size_t)w * steps + k] = h;
        }
    }
    wait_store(x, row, count, fixture);
}

int validate(int n, int max_m, const D1Config *c, const D1Tables *t) {
    if (n < 0 || max_m < 1 || max_m > D1_MAX_MONSTERS || !c || !t || !t->ray_slots) return D1_E_ARG;
    if (t->nslots < 1 || t->nslots > 64) return D1_E_ARG;
    if (c->count < 1 || c->count > max_m) return D1_E_CONFIG;
    if (c->rng_mode < 0 || c->rng_mode > 1 || c->level_mode < 0 || c->level_mode > 1) return D1_E_CONFIG;
    if (c->level_mode == 0 && (!t->floor || !t->cells)) return D1_E_ARG;
    if (c->roster_mode < 0 || c->roster_mode > 1 || (c->stairs != 0 && c->stairs != 3)) return D1_E_CONFIG;
    if (c->roster_mode == 1 && (c->hp_lo < 1 || c->hp_hi < c->hp_lo || c->hp_hi > 30000)) return D1_E_CONFIG;
    if (c->hp < 1 || c->hp > 30000 || c->ac100 < 0 || c->ev100 < 0 || c->sh100 < 0 || c->limit < 1) return D1_E_CONFIG;
    for (int k = 0; k < 6; k++)
        if (c->kinds[k].speed < 0 || c->kinds[k].speed > 20 || c->kinds[k].damage < 0 || c->kinds[k].tohit < 0 ||
            c->kinds[k].bypass < 0)
            return D1_E_CONFIG;
    return 0;
}

}  // namespace d1

extern "C" {
int d1_state_bytes(int max_monsters) {
    if (max_monsters < 1 || max_monsters > D1_MAX_MONSTERS) return D1_E_ARG;
    return d1::state_bytes(max_monsters);
}
int d1_obs_bytes(void) { return D1_OBS_BYTES; }
int d1_action_size(void) { return D1_ACTIONS; }
int d1_out_size(void) { return D1_OUT; }
int d1_config_bytes(void) { return (int)sizeof(D1Config); }

int d1_wait_bytes(void) { return d1::WAIT_BYTES; }
static int wait_validate(int n, int count, const D1Config *cfg, const D1WaitMap *map) {
    if (n < 0 || count < 0 || count > 64 || !cfg || !map || !map->floor || !map->dist || !map->starts) return D1_E_ARG;
    if (map->player < 0 || map->player >= D1_N) return D1_E_ARG;
    for (int k = 0; k < 6; k++)
        if (cfg->kinds[k].speed < 0 || cfg->kinds[k].speed > 20) return D1_E_CONFIG;
    return 0;
}
int d1_wait_init(void *worlds, int n, int count, const D1Config *cfg, const D1WaitMap *map, uint64_t seed,
                 int scenario, void *stream) {
    int e = wait_validate(n, count, cfg, map);
    if (e) return e;
    if (!worlds || scenario < 0 || scenario > 2) return D1_E_ARG;
    if (n == 0) return 0;
    hipLaunchKernelGGL(d1::k_wait_init, dim3(n), dim3(64), 0, (hipStream_t)stream, (uint8_t *)worlds, n, count,
                       *cfg, *map, seed, scenario);
    return (int)hipGetLastError();
}
int d1_wait_run(void *worlds, int n, int count, const D1Config *cfg, const D1WaitMap *map, int steps,
                uint32_t *trace, void *stream) {
    int e = wait_validate(n, count, cfg, map);
    if (e) return e;
    if (!worlds || steps < 0) return D1_E_ARG;
    if (n == 0 || steps == 0) return 0;
    hipLaunchKernelGGL(d1::k_wait, dim3(n), dim3(64), 0, (hipStream_t)stream, (uint8_t *)worlds, n, count, *cfg,
                       *map, steps, trace);
    return (int)hipGetLastError();
}
int d1_init(void *state, int n, int max_monsters, const D1Config *cfg, const D1Tables *tab, uint64_t seed,
            uint8_t *obs, uint32_t *hash, void *stream) {
    int e = d1::validate(n, max_monsters, cfg, tab);
    if (e) return e;
    if (!state) return D1_E_ARG;
    if (n == 0) return 0;
    hipLaunchKernelGGL(d1::k_init, dim3(n), dim3(64), 0, (hipStream_t)stream, (uint8_t *)state, n, max_monsters,
                       (size_t)d1::state_bytes(max_monsters), *cfg, *tab, seed, obs, hash);
    return (int)hipGetLastError();
}
int d1_step(void *state, int n, int max_monsters, const D1Config *cfg, const D1Tables *tab, const int64_t *actions,
            uint8_t *obs, float *out, uint32_t *hash, const uint8_t *active, void *stream) {
    int e = d1::validate(n, max_monsters, cfg, tab);
    if (e) return e;
    if (!state || !actions) return D1_E_ARG;
    if (n == 0) return 0;
    hipLaunchKernelGGL(d1::k_step, dim3(n), dim3(64), 0, (hipStream_t)stream, (uint8_t *)state, n, max_monsters,
                       (size_t)d1::state_bytes(max_monsters), *cfg, *tab, actions, obs, out, hash, active);
    return (int)hipGetLastError();
}
}
