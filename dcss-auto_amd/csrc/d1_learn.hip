// d1learn: the reference's d1-stairs-v2 learning task behind its learn_* C ABI
// (include/d1learn.h), for MI355X (gfx950).
//
// One wavefront owns one world per launch, as in d1_env.hip, and reuses its device
// core (d1_core.h: RNG, LDS bitmaps, melee, monster pathing, distance field). What
// this task adds, all wave-parallel:
//   * player view and monster waking read the caller's per-map LOS table
//     (10 dwords per origin); four ballots give the view's quadrant sets;
//   * the frontier-anchor list keeps the reference's order exactly. A reveal can
//     only change anchors in the 17x17 window around the player; the changed cells
//     are applied in the order the reference's refresh loop first touches them
//     (key = position in the "each newly viewed cell, then its eight neighbours"
//     sequence, taken by wave-min), appended or swap-removed through a per-window
//     position table. The list is worked on in place in the state row (through the
//     caches: staging it in LDS and writing its changed part back cost more);
//   * the known-floor BFS (viewed floor, from the player) is bit-parallel over LDS
//     rows and stops once the nearest anchor layer and every remembered stair (or
//     visible enemy, for the controller) is reached; route cues walk it backwards;
//   * the fp32 observation [1015] is staged in LDS and written coalesced; the mask
//     [19] and outcome [45] by one lane each.
// Task constants are those of gpu-d1/branches/d1-stairs-v2/scripts/assets.py:5.
// D1_CLUMP_MODE (0 or 1) selects the reset's clumped placement, as the reference's
// CLUMP_MODE build flag does.
#include "../../include/d1learn.h"

#define D1_STAGE_FLOATS D1L_OBS   // the fp32 observation is staged over the dead BFS bitmaps
#include "d1_core.h"

#ifndef D1_CLUMP_MODE
#define D1_CLUMP_MODE 0
#endif

namespace d1 {
namespace learn {

constexpr int LE = D1L_ENEMIES, REQ = D1L_REQUIRED;
// observation offsets (gpu-d1/branches/d1-stairs-v2/src/learn.cu:101-112)
constexpr int O_ENEMY_HP = 225, O_RECORDS = 450, O_PLAYER = 650, O_RING = 654, O_FRONTIER = 718, O_VISIBLE = 733,
              O_PROGRESS = 958, O_SLEEP = 959, O_STAIR = 999;
constexpr int CLEAR_MILLI = 1000;
constexpr float TURN_COST = 0.00001f;
constexpr int WIN = 17;      // 17x17 window in which a reveal can change anchors
constexpr int INF = 0x7FFFFFFF;

// ---------------------------------------------------------------- state row
struct LHdr {
    uint64_t rng_state, rng_inc, encountered;   // PCG32; bit i = enemy i seen at least once
    int32_t ticks, killed, decisions, floor_seen, episode, first_stair_tick;
    int16_t player, hp, regen, blocks, map_id, next_slot, frontier_count, stairs[3];
    uint8_t clumped, error, pad[10];
};
static_assert(sizeof(LHdr) == 80, "learn header layout");
struct LMon {
    int16_t pos, hp, energy;
    uint8_t awake;
    int8_t slot;   // encounter slot, -1 before the first sighting
};
static_assert(sizeof(LMon) == 8, "learn monster layout");
constexpr int OFF_MON = 80, OFF_VIEWED = OFF_MON + 8 * REQ, OFF_FLOOR = OFF_VIEWED + ROWS_WORDS * 4,
              OFF_LIST = OFF_FLOOR + ROWS_WORDS * 4;
constexpr int ROW_BYTES = (OFF_LIST + 2 * N + 63) / 64 * 64;

struct LSmem {
    Smem s;                       // floor, viewed, occ (living enemies), reach, front, dist
    uint32_t anch[ROWS_WORDS];    // frontier anchors (then: anchors of the nearest BFS layer)
    int16_t wslot[WIN * WIN];     // list position of anchors inside the window
    int32_t cbase[16];            // rank of the first newly viewed cell of each view row
};

struct LCtx {
    Ctx x;
    LSmem *L;
    const D1LTables *t;
    const uint32_t *los;   // this map's LOS rows
    int map_id, next_slot, nf;   // nf = frontier list length
    uint64_t enc;
    int mslot;             // this lane's enemy slot
    uint16_t *lst;         // the row's frontier list
    int clumped, error;
};

__device__ __forceinline__ Row row_xor(Row x, Row y) { return {x.a ^ y.a, x.b ^ y.b, x.c ^ y.c}; }
__device__ __forceinline__ int lanes_below(uint64_t m, int lane) {
    return __popcll(m & ((1ULL << lane) - 1ULL));
}
__device__ __forceinline__ bool floor_b(const LCtx &c, int p) { return p >= 0 && bit(c.x.sm->floor, p); }

// ---------------------------------------------------------------- view from the LOS table
// in_view (learn.cu:192-198): bit (dy+8)*17+dx+8 of the player's LOS row; lane j
// tests offset (j%8, j/8) of each quadrant.
__device__ __forceinline__ uint32_t los_bit(const uint32_t *row, int dx, int dy) {
    int b = (dy + 8) * 17 + dx + 8;
    return (row[b >> 5] >> (b & 31)) & 1u;
}
__device__ __forceinline__ void view_los(LCtx &c) {
    Ctx &x = c.x;
    const uint32_t *row = c.los + (size_t)x.player * 10;
    int px = x.player % W, py = x.player / W, tx = x.lane & 7, ty = x.lane >> 3;
    set_view(x, ballot(los_bit(row, tx, ty) && inb(px + tx, py + ty)), ballot(los_bit(row, -tx, ty) && inb(px - tx, py + ty)),
             ballot(los_bit(row, -tx, -ty) && inb(px - tx, py - ty)), ballot(los_bit(row, tx, -ty) && inb(px + tx, py - ty)));
}
// monster_detects_player (learn.cu:201-207) for this lane's monster
__device__ __forceinline__ bool lane_detects(const LCtx &c, int origin) {
    int dx = c.x.player % W - origin % W, dy = c.x.player / W - origin / W;
    if (iabs(dx) > 6 || iabs(dy) > 6) return false;
    return los_bit(c.los + (size_t)origin * 10, dx, dy);
}
__device__ __forceinline__ bool lane_alive(const LCtx &c) { return c.x.lane < REQ && c.x.mhp > 0; }
__device__ __forceinline__ bool visible_enemy(const LCtx &c) {
    return ballot(lane_alive(c) && in_view(c.x, c.x.mpos)) != 0;
}
// update_knowledge (learn.cu:212-218): sighted enemies are encountered and take the
// next free slots in index order.
__device__ __forceinline__ void update_knowledge(LCtx &c) {
    bool vis = lane_alive(c) && in_view(c.x, c.x.mpos);
    c.enc |= ballot(vis);
    uint64_t need = ballot(vis && c.mslot < 0);
    if (vis && c.mslot < 0) c.mslot = c.next_slot + lanes_below(need, c.x.lane);
    c.next_slot += __popcll(need);
}

// ---------------------------------------------------------------- frontier anchors
// Seen floor (viewed floor) with an in-bounds neighbour never viewed
// (FRONTIER_RING_MEMORY_WALLS_OBS rule, learn.cu:269-280).
__device__ __forceinline__ Row anchor_row(const Smem *sm, int y) {
    const Row all = row_range(0, W - 1);
    Row u{0, 0, 0};
    for (int yy = y - 1; yy <= y + 1; yy++)
        if (yy >= 0 && yy < H) u = row_or(u, row_andn(all, row_ld(sm->viewed, yy)));
    u = row_and(row_or(u, row_or(row_shl1(u), row_shr1(u))), all);
    return row_and(row_and(row_ld(sm->floor, y), row_ld(sm->viewed, y)), u);
}
__device__ __forceinline__ void anchors_all(LCtx &c) {
    for (int y = c.x.lane; y < H; y += 64) row_st(c.L->anch, y, anchor_row(c.x.sm, y));
    __syncthreads();
}
__device__ __forceinline__ int popc_below(Row r, int xx) {
    if (xx < 32) return __popc(r.a & ((1u << xx) - 1u));
    if (xx < 64) return __popc(r.a) + __popc(r.b & ((1u << (xx - 32)) - 1u));
    return __popc(r.a) + __popc(r.b) + __popc(r.c & ((1u << (xx - 64)) - 1u));
}

// reveal (learn.cu:298-336): mark the view, count fresh floor, then replay the
// frontier refreshes in the reference's order.
__device__ __forceinline__ int reveal_learn(LCtx &c) {
    Ctx &x = c.x;
    Smem *sm = x.sm;
    LSmem *L = c.L;
    view_los(c);
    const int px = x.player % W, py = x.player / W;
    const int wy0 = py - 8, wx0 = px - 8;
    const int ya = wy0 + x.lane;
    const bool arow = x.lane < WIN && ya >= 0 && ya < H;
    Row a0{0, 0, 0};
    if (arow) a0 = anchor_row(sm, ya);
    // view rows py-7..py+7 (lane l < 15)
    int dy = x.lane - 7, y = py + dy, fresh = 0, cnt = 0;
    bool mine = x.lane < 15 && y >= 0 && y < H;
    Row mask{0, 0, 0}, chg{0, 0, 0}, old{0, 0, 0};
    if (mine) {
        int ay = iabs(dy);
        uint32_t R = 0, Lf = 0;
        if (dy >= 0) { R |= (uint32_t)(view_q(x, 0) >> (8 * ay)) & 0xFFu; Lf |= (uint32_t)(view_q(x, 1) >> (8 * ay)) & 0xFFu; }
        if (dy <= 0) { R |= (uint32_t)(view_q(x, 3) >> (8 * ay)) & 0xFFu; Lf |= (uint32_t)(view_q(x, 2) >> (8 * ay)) & 0xFFu; }
        uint32_t v15 = (__builtin_bitreverse32(Lf) >> 24) | (R << 7);
        mask = row_place15(v15, px);
        old = row_ld(sm->viewed, y);
        chg = row_andn(mask, old);
        fresh = row_popc(row_and(chg, row_ld(sm->floor, y)));
        cnt = row_popc(chg);
    }
    int pre = cnt;   // inclusive prefix over view rows
    for (int o = 1; o < 16; o <<= 1) { int v = __shfl_up(pre, o); if (x.lane >= o) pre += v; }
    __syncthreads();
    if (mine) { row_st(sm->viewed, y, row_or(mask, old)); row_st(sm->front, y, chg); }
    if (x.lane < 15) L->cbase[x.lane] = pre - cnt;
    __syncthreads();
    Row a1{0, 0, 0};
    if (arow) a1 = anchor_row(sm, ya);
    __syncthreads();
    if (arow) { row_st(sm->reach, ya, row_xor(a0, a1)); row_st(L->anch, ya, a1); }
    // list positions of anchors inside the window
    for (int j = x.lane; j < c.nf; j += 64) {
        int p = c.lst[j], wx = p % W - wx0, wy = p / W - wy0;
        if (wx >= 0 && wx < WIN && wy >= 0 && wy < WIN) L->wslot[wy * WIN + wx] = (int16_t)j;
    }
    __syncthreads();
    // key of each changed window cell: its first position in the refresh sequence
    auto in_chg = [&](int qx, int qy) -> bool {
        return qx >= px - 7 && qx <= px + 7 && qy >= py - 7 && qy <= py + 7 && inb(qx, qy) && bit_at(sm->front, qx, qy);
    };
    auto rank = [&](int qx, int qy) -> int {
        return L->cbase[qy - (py - 7)] + popc_below(row_ld(sm->front, qy), qx);
    };
    int key[5];
    int adds = 0;
#pragma unroll
    for (int k = 0; k < 5; k++) {
        int w = x.lane + 64 * k, qx = wx0 + w % WIN, qy = wy0 + w / WIN;
        key[k] = INF;
        if (w < WIN * WIN && inb(qx, qy) && bit_at(sm->reach, qx, qy)) {
            int kk = in_chg(qx, qy) ? 9 * rank(qx, qy) : INF;
#pragma unroll
            for (int d = 0; d < 8; d++) {
                int ddx = d == 1 || d == 4 || d == 5 ? 1 : d == 3 || d == 6 || d == 7 ? -1 : 0;
                int ddy = d == 0 || d == 4 || d == 7 ? -1 : d == 2 || d == 5 || d == 6 ? 1 : 0;
                int cx = qx - ddx, cy = qy - ddy;   // q = neighbor(c, d)
                if (in_chg(cx, cy)) kk = imin(kk, 9 * rank(cx, cy) + 1 + d);
            }
            key[k] = kk;
            adds += bit_at(L->anch, qx, qy);
        }
    }
    adds = (int)wave_sum((uint32_t)adds);
    uint16_t *lst = c.lst;
    int nf = c.nf;
    for (;;) {
        int lm = imin(imin(imin(key[0], key[1]), imin(key[2], key[3])), key[4]);
        int m = wave_min(lm);
        if (m == INF) break;
        int wl = __ffsll((unsigned long long)ballot(lm == m)) - 1;
        int wc = key[0] == m ? x.lane : key[1] == m ? x.lane + 64 : key[2] == m ? x.lane + 128
               : key[3] == m ? x.lane + 192 : x.lane + 256;
        wc = lane_val(wc, wl);
        if (x.lane == wl) {
#pragma unroll
            for (int k = 0; k < 5; k++) key[k] = key[k] == m ? INF : key[k];
        }
        int q = (wy0 + wc / WIN) * W + wx0 + wc % WIN;
        // every lane performs the same uniform update, so each sees its own writes
        if (bit(L->anch, q)) {
            if (nf >= N) { c.error = 1; continue; }
            lst[nf] = (uint16_t)q;
            L->wslot[wc] = (int16_t)nf;
            nf++;
        } else {
            int s = L->wslot[wc];
            if (s < 0 || s >= nf) { c.error = 1; continue; }
            int last = --nf;
            int r = lst[last];
            lst[s] = (uint16_t)r;
            int rx = r % W - wx0, ry = r / W - wy0;
            if (rx >= 0 && rx < WIN && ry >= 0 && ry < WIN) L->wslot[ry * WIN + rx] = (int16_t)s;
        }
    }
    __threadfence_block();
    c.nf = nf;
    __syncthreads();
    int total = (int)wave_sum((uint32_t)fresh);
    x.floor_seen += total;
    return total;
}

// ---------------------------------------------------------------- reset (learn.cu:351-446)
// Reservoir choice over the map's cell list in list order (count c kept when
// r(c) == 0, the last kept wins): the eligible count, the shared parallel reservoir
// draw, then the chosen eligible cell.
template <class Pred>
__device__ __forceinline__ int reservoir_cells(LCtx &c, Rng &g, const int16_t *cells, int ncells, Pred pred) {
    int total = 0;
    for (int j0 = 0; j0 < ncells; j0 += 64) {
        int j = j0 + c.x.lane;
        int p = j < ncells ? (int)cells[j] : -1;
        total += __popcll(ballot(p >= 0 && p < N && pred(p)));
    }
    int k = reservoir(g, total, c.x.lane);
    if (k < 0) return -1;
    for (int j0 = 0; j0 < ncells; j0 += 64) {
        int j = j0 + c.x.lane;
        int p = j < ncells ? (int)cells[j] : -1;
        uint64_t m = ballot(p >= 0 && p < N && pred(p));
        int cnt = __popcll(m);
        if (k < cnt) return lane_val(p, select64(m, k));
        k -= cnt;
    }
    return -1;
}
// A cell from the map's list; an entry outside the grid (a bad table) reads as cell 0
// and marks the world's error flag instead of indexing out of bounds.
__device__ __forceinline__ int cell_at(LCtx &c, const int16_t *cells, int k) {
    int p = cells[k];
    if (p < 0 || p >= N) { c.error = 1; p = 0; }
    return p;
}
__device__ __forceinline__ int free_floor(const LCtx &c, int q) {
    return q >= 0 && bit(c.x.sm->floor, q) && q != c.x.player && !bit(c.x.sm->occ, q);
}

template <int CLUMP>
__device__ __forceinline__ void reset_learn(LCtx &c) {
    Ctx &x = c.x;
    Smem *sm = x.sm;
    const D1Config *cf = x.c;
    const D1LTables &t = *c.t;
    c.map_id = t.map_filter >= 0 ? t.map_filter : x.g.r(t.n_maps);
    const int m = c.map_id;
    int ncells = t.map_ncells[m];
    if (ncells < 1 || ncells > N) { c.error = 1; ncells = imin(imax(ncells, 1), N); }
    const int16_t *cells = t.cells + (size_t)m * N;
    c.los = t.los + (size_t)m * N * 10;
    // this map's floor bitmap (rows lane, lane+64) from the byte map
    const uint32_t *fb = (const uint32_t *)(t.floor + (size_t)m * N);
    for (int yy = x.lane; yy < H; yy += 64) {
        uint32_t w[3] = {0, 0, 0};
        for (int k = 0; k < 20; k++) {
            uint32_t v = fb[yy * 20 + k];
#pragma unroll
            for (int b = 0; b < 4; b++) {
                int xx = 4 * k + b;
                uint32_t on = ((v >> (8 * b)) & 0xFFu) != 0;
                if (xx < 32) w[0] |= on << xx;
                else if (xx < 64) w[1] |= on << (xx - 32);
                else w[2] |= on << (xx - 64);
            }
        }
        row_st(sm->floor, yy, Row{w[0], w[1], w[2]});
    }
    for (int wd = x.lane; wd < ROWS_WORDS; wd += 64) { sm->occ[wd] = 0; sm->viewed[wd] = 0; }
    __syncthreads();
    x.player = cell_at(c, cells, x.g.r(ncells));
    x.hp = cf->hp; x.regen = 0; x.blocks = 0;
    x.ticks = 0; x.decisions = 0; x.killed = 0; x.floor_seen = 0;
    c.next_slot = 0; c.enc = 0; c.mslot = -1;
    const int MHP[6] = {8, 10, 12, 16, 12, 10};
    int mpos = -1, men = -30000;
    for (int i = 0; i < REQ; i++) {
        int p = 0, tries = 0;
        do {
            p = cell_at(c, cells, x.g.r(ncells));
        } while ((p == x.player || bit(sm->occ, p)) && ++tries < (1 << 20));
        if (p == x.player || bit(sm->occ, p)) c.error = 1;
        occ_set(x, p, true);
        int en = 70 + x.g.r(10);
        if (x.lane == i) { mpos = p; men = en; }
    }
    x.mpos = x.lane < REQ ? mpos : -1;
    x.mhp = x.lane < REQ ? MHP[x.lane % 6] : 0;
    x.menergy = x.lane < REQ ? men : -30000;
    x.mawake = 0;
    x.mkind = x.lane % 6;
    // clumps of three from a copy of the RNG (learn.cu:379-402)
    Rng place = x.g;
    c.clumped = CLUMP == 2 || (CLUMP == 1 && place.r(3) == 0);
    if (c.clumped) {
        for (int wd = x.lane; wd < ROWS_WORDS; wd += 64) sm->occ[wd] = 0;
        __syncthreads();
        for (int i = 0; i < REQ; i += 3) {
            int anchor = reservoir_cells(c, place, cells, ncells, [&](int p) {
                if (p == x.player || bit(sm->occ, p)) return false;
                int fr = 0;
                for (int a = 0; a < 8; a++) fr += free_floor(c, nbr(p, a));
                return fr >= 2;
            });
            if (anchor < 0) { c.error = 1; break; }
            occ_set(x, anchor, true);
            if (x.lane == i) x.mpos = anchor;
            for (int k = 1; k <= 2; k++) {
                int chosen = -1, nn = 0;
                for (int a = 0; a < 8; a++) {
                    int q = nbr(anchor, a);
                    if (free_floor(c, q) && place.r(++nn) == 0) chosen = q;
                }
                if (chosen < 0) { c.error = 1; break; }
                occ_set(x, chosen, true);
                if (x.lane == i + k) x.mpos = chosen;
            }
        }
    }
    // three stairs from another copy (learn.cu:422-441)
    Rng st = x.g;
    x.first_stair_tick = -1;
    x.stairs = pack_stairs(-1, -1, -1);
    for (int k = 0; k < 3; k++) {
        uint64_t prev = x.stairs;
        int sel = reservoir_cells(c, st, cells, ncells, [&](int p) {
            bool ok = cheb(p, x.player) >= 12 && !bit(sm->occ, p);
            for (int q = 0; q < k; q++) ok = ok && cheb(p, (int16_t)(uint16_t)(prev >> (16 * q))) >= 8;
            return ok;
        });
        if (sel < 0) c.error = 1;
        x.stairs = (x.stairs & ~(0xFFFFULL << (16 * k))) | (uint64_t)(uint16_t)sel << (16 * k);
    }
    c.nf = 0;
    reveal_learn(c);   // the initial view earns no reward
    update_knowledge(c);
}

// ---------------------------------------------------------------- known-floor BFS (learn.cu:222-266)
// Bit-parallel BFS over viewed floor from the player into sm->reach and the layer-mod-3
// planes sm->lay0/lay1. Stops when the first layer holding an anchor is found (its anchors then
// replace L->anch), every wanted stair has a layer and every wanted monster lane is
// reached, or nothing new is reached. Returns the anchor layer or -1.
struct KB {
    int alayer;
    int sl0, sl1, sl2;   // stair layers, -1 = not reached
    int mlayer;          // this lane's monster layer
};
// Lane l keeps rows l and (l < 6) 64 + l of the frontier, reach, known floor and anchors in
// registers; vertical neighbours arrive by lane shuffles, so a layer needs no LDS round
// trip and no barrier. Reach, the layer planes, the last layer's frontier and the anchor
// rows are published at the end.
__device__ __forceinline__ uint32_t row_word(Row r, int w) { return w == 0 ? r.a : w == 1 ? r.b : r.c; }
__device__ __forceinline__ KB known_bfs(LCtx &c, bool want_anchor, int want_stairs, bool want_monster) {
    Ctx &x = c.x;
    Smem *sm = x.sm;
    LSmem *L = c.L;
    const int lane = x.lane;
    const bool has1 = lane < H - 64;
    const Row zero{0, 0, 0};
    KB r{-1, -1, -1, -1, -1};
    __syncthreads();   // floor, viewed and anchor rows written by other lanes
    const Row k0 = row_and(row_ld(sm->floor, lane), row_ld(sm->viewed, lane));
    const Row k1 = has1 ? row_and(row_ld(sm->floor, 64 + lane), row_ld(sm->viewed, 64 + lane)) : zero;
    Row a0 = zero, a1 = zero;
    if (want_anchor) {
        a0 = row_ld(L->anch, lane);
        if (has1) a1 = row_ld(L->anch, 64 + lane);
    }
    const int py = x.player / W, px = x.player % W;
    const Row pbit = row_range(px, px);
    Row f0 = lane == py ? pbit : zero, f1 = has1 && 64 + lane == py ? pbit : zero;
    Row r0 = f0, r1 = f1;
    Row e0 = zero, e1 = zero, g0 = zero, g1 = zero;   // layer % 3 == 1, layer % 3 == 2
    int m3 = 0;
    // wanted stairs: holder lane, register row and word of each (uniform)
    const int s0 = stair_at(x, 0), s1 = stair_at(x, 1), s2 = stair_at(x, 2);
    // this lane's monster cell, when it is wanted: holder lane and word of its row
    const bool mneed = want_monster && lane_alive(c) && in_view(x, x.mpos);
    const int my = mneed ? x.mpos / W : 0, mx = mneed ? x.mpos % W : 0;
    const int msrc = my & 63, mword = mx >> 5;
    const uint32_t mbit = 1u << (mx & 31);
    for (int layer = 0; layer < N; layer++) {
        if (layer > 0) {
            const Row f1_0 = row_lane(f1, 0), f0_63 = row_lane(f0, 63);
            const Row u0 = row_sel(lane == 0, zero, row_up(f0)), d0 = row_sel(lane == 63, f1_0, row_dn(f0));
            const Row u1 = row_sel(lane == 0, f0_63, row_up(f1)), d1 = row_sel(lane >= H - 65, zero, row_dn(f1));
            const Row n0 = row_andn(row_and(dilate(f0, u0, d0), k0), r0);
            const Row n1 = has1 ? row_andn(row_and(dilate(f1, u1, d1), k1), r1) : zero;
            r0 = row_or(r0, n0); r1 = row_or(r1, n1);
            f0 = n0; f1 = n1;
            m3 = m3 == 2 ? 0 : m3 + 1;
            if (m3 == 1) { e0 = row_or(e0, n0); e1 = row_or(e1, n1); }
            if (m3 == 2) { g0 = row_or(g0, n0); g1 = row_or(g1, n1); }
            if (!ballot(row_any(n0) || row_any(n1))) break;
        }
        bool done = true;
        if (want_anchor && r.alayer < 0) {
            const Row h0 = row_and(f0, a0), h1 = row_and(f1, a1);
            if (ballot(row_any(h0) || row_any(h1))) {
                r.alayer = layer;
                a0 = h0; a1 = h1;
            } else done = false;
        }
#define D1_STAIR_LAYER(bitmask, st, sl)                                                                       \
        if (want_stairs & (bitmask)) {                                                                        \
            if (sl < 0) {                                                                                     \
                const int sy = (st) / W, sx = (st) % W;                                                      \
                const uint32_t w = (uint32_t)lane_val((int)row_word(sy >= 64 ? r1 : r0, sx >> 5), sy & 63); \
                if ((w >> (sx & 31)) & 1u) sl = layer;                                                        \
            }                                                                                                 \
            done = done && sl >= 0;                                                                           \
        }
        D1_STAIR_LAYER(1, s0, r.sl0)
        D1_STAIR_LAYER(2, s1, r.sl1)
        D1_STAIR_LAYER(4, s2, r.sl2)
#undef D1_STAIR_LAYER
        if (want_monster) {
            if (ballot(mneed && r.mlayer < 0)) {
                const Row q0 = {(uint32_t)__shfl((int)r0.a, msrc), (uint32_t)__shfl((int)r0.b, msrc), (uint32_t)__shfl((int)r0.c, msrc)};
                const Row q1 = {(uint32_t)__shfl((int)r1.a, msrc), (uint32_t)__shfl((int)r1.b, msrc), (uint32_t)__shfl((int)r1.c, msrc)};
                const uint32_t w = row_word(my >= 64 ? q1 : q0, mword);
                if (mneed && r.mlayer < 0 && (w & mbit)) r.mlayer = layer;
                if (ballot(mneed && r.mlayer < 0)) done = false;
            }
        }
        if (done) break;
    }
    row_st(sm->reach, lane, r0);
    row_st(sm->front, lane, f0);
    row_st(sm->lay0, lane, e0);
    row_st(sm->lay1, lane, g0);
    if (has1) {
        row_st(sm->reach, 64 + lane, r1); row_st(sm->front, 64 + lane, f1);
        row_st(sm->lay0, 64 + lane, e1); row_st(sm->lay1, 64 + lane, g1);
    }
    if (want_anchor) {   // the nearest layer's anchors; none reachable: the set is not needed
        row_st(L->anch, lane, r.alayer >= 0 ? a0 : zero);
        if (has1) row_st(L->anch, 64 + lane, r.alayer >= 0 ? a1 : zero);
    }
    __syncthreads();
    return r;
}
// route_first_step (learn.cu:248-264): back from target (at layer D) along the first
// predecessor in direction order; the player's direction to the layer-1 cell. A reached
// neighbour of a layer-D cell is at layer D-1 exactly when its layer mod 3 is (D-1) mod 3
// (neighbours differ by at most one layer).
__device__ __forceinline__ int route_first_step(const LCtx &c, int target, int D) {
    const Ctx &x = c.x;
    const Smem *sm = x.sm;
    if (target < 0 || D < 0 || target == x.player) return -1;
    int p = target;
    for (; D > 1; D--) {
        int q = nbr(p, x.lane & 7);
        bool ok = x.lane < 8 && q >= 0 && bit(sm->reach, q) && lay3(sm, q) == (D - 1) % 3;
        uint64_t mm = ballot(ok);
        if (!mm) return -1;
        p = lane_val(q, __ffsll((unsigned long long)mm) - 1);
    }
    uint64_t mm = ballot(x.lane < 8 && nbr(x.player, x.lane & 7) == p);
    return mm ? __ffsll((unsigned long long)mm) - 1 : -1;
}
// First frontier-list entry in the nearest anchor layer (the reference's first
// strict minimum over the list).
__device__ __forceinline__ int first_hit(const LCtx &c) {
    for (int j0 = 0; j0 < c.nf; j0 += 64) {
        int j = j0 + c.x.lane;
        int p = j < c.nf ? (int)c.lst[j] : 0;
        uint64_t mm = ballot(j < c.nf && p < N && bit(c.L->anch, p));
        if (mm) return lane_val(p, __ffsll((unsigned long long)mm) - 1);
    }
    return -1;
}
__device__ __forceinline__ int known_stairs_l(const Ctx &x) { return known_stairs(x); }
// seen-stair mask (bit k)
__device__ __forceinline__ int seen_stairs(const Ctx &x) {
    int m = 0;
    for (int k = 0; k < 3; k++) m |= (stair_at(x, k) >= 0 && seen_at(x, stair_at(x, k))) << k;
    return m;
}
// nearest_stair (learn.cu:345-350) from the BFS stair layers; layer into D
__device__ __forceinline__ int nearest_stair(const Ctx &x, int seen, const KB &r, int &D) {
    int best = -1;
    D = 65535;
    int l[3] = {r.sl0, r.sl1, r.sl2};
#pragma unroll
    for (int k = 0; k < 3; k++)
        if (((seen >> k) & 1) && l[k] >= 0 && l[k] < D) { best = stair_at(x, k); D = l[k]; }
    return best;
}

// ---------------------------------------------------------------- one physical turn (learn.cu:684-828)
struct POut {
    float reward;
    int done, clear, death, timeout, killed, hp, ticks;
    int enc, alive_unenc, alive_enc, vis, floor_seen, ncells, known, first_tick, stair;
    int saw_enemy, saw_awake;
};

template <int CLUMP>
__device__ __forceinline__ void primitive_learn(LCtx &c, int d, int limit, POut &o) {
    Ctx &x = c.x;
    Smem *sm = x.sm;
    const D1Config *cf = x.c;
    int milli = 0;
    x.blocks = 0;
    x.regen += cf->regen;
    while (x.regen >= 100) { x.hp = imin(cf->hp, x.hp + 1); x.regen -= 100; }
    if (d >= 0 && d < 8) {
        int p = nbr(x.player, d);
        if (p >= 0 && bit(sm->floor, p)) {
            uint64_t at = ballot(lane_alive(c) && x.mpos == p);
            if (at) {
                int id = __ffsll((unsigned long long)at) - 1;
                c.enc |= 1ULL << id;
                int sl = lane_val(c.mslot, id);
                if (sl < 0) { if (x.lane == id) c.mslot = c.next_slot; c.next_slot++; }
                if (x.g.r(5) != 0) {
                    int nh = (int16_t)(lane_val(x.mhp, id) - (1 + x.g.r(4)));
                    if (nh <= 0) {
                        if (x.lane == id) { x.mhp = 0; x.menergy = -30000; }
                        occ_set(x, p, false);
                        x.killed++;
                    } else if (x.lane == id) x.mhp = nh;
                }
            } else x.player = p;
        }
    }
    reveal_learn(c);   // EXPLORE_MILLI = 0, the reveal still updates memory
    o.saw_awake = visible_awake(x);
    o.saw_enemy = visible_enemy(c);
    const bool clear = d == 18 && stair_index(x) > 0 && x.hp > 0;
    if (!clear) {
        bool alive = lane_alive(c);
        bool wake = alive && !x.mawake && lane_detects(c, x.mpos);
        if (wake) { x.mawake = 1; x.menergy = 70; }
        if (alive && !x.mawake) x.menergy = -30000;
        if (alive) x.menergy = (int16_t)(x.menergy + kind_speed(cf, x.mkind));
        int maxspeed = 0;
        for (int k = 0; k < 6; k++) maxspeed = imax(maxspeed, cf->kinds[k].speed);
        uint64_t movers = ballot(alive && x.mawake && x.menergy >= 80 && cheb(x.mpos, x.player) > 1);
        if (movers) bfs(x, movers, imax(2, (maxspeed + 9) / 10));
        while (x.hp > 0 && ballot(x.lane < REQ && x.menergy >= 80)) {   // no reduction once nobody can act
            // the lane id opaque per act, so that the monster rules' lane-derived masks and
            // addresses are recomputed in each act instead of held through the loop: 168 -> 121
            // VGPRs, 3 -> 4 waves per SIMD, k_learn_step 0.903 -> 0.796 ms
            {
                int l = lane_id();
                asm volatile("" : "+v"(l));
                x.lane = l;
            }
            const int key = wave_max(x.lane < REQ && x.menergy >= 80 ? x.menergy * 128 + 127 - x.lane : -1);
            int id = 127 - (key & 127);
            act(x, id);
            if (!(o.saw_enemy && o.saw_awake) && in_view(x, lane_val(x.mpos, id))) {   // nothing left to learn once both are set
                o.saw_enemy = 1;
                if (lane_val(x.mawake, id)) o.saw_awake = 1;
            }
        }
    }
    x.ticks++;
    if (x.first_stair_tick < 0 && known_stairs(x) > 0) x.first_stair_tick = x.ticks;
    const bool death = x.hp <= 0, timeout = !clear && !death && x.ticks >= limit;
    if (clear) milli += CLEAR_MILLI;
    float reward = 0.001f * (float)milli;
    reward -= TURN_COST;
    o.saw_enemy = o.saw_enemy || visible_enemy(c);
    o.saw_awake = o.saw_awake || visible_awake(x);
    update_knowledge(c);
    bool alive = lane_alive(c), enc = x.lane < REQ && ((c.enc >> x.lane) & 1);
    o.enc = __popcll(c.enc & ((1ULL << REQ) - 1ULL));
    o.alive_unenc = __popcll(ballot(alive && !enc));
    o.alive_enc = __popcll(ballot(alive && enc));
    o.vis = __popcll(ballot(alive && in_view(x, x.mpos)));
    o.floor_seen = x.floor_seen;
    o.ncells = c.t->map_ncells[c.map_id];
    o.known = known_stairs(x);
    o.first_tick = x.first_stair_tick;
    o.stair = clear ? stair_index(x) : 0;
    o.reward = reward;
    o.done = clear || death || timeout;
    o.clear = clear; o.death = death; o.timeout = timeout;
    o.killed = x.killed; o.hp = imax(0, x.hp); o.ticks = x.ticks;
    if (o.done) { x.episode++; reset_learn<CLUMP>(c); }
}

// The later turns of a REST whose first turn left no living monster awake. Each repeats that
// turn (learn.cu:684-828 with a WAIT) except for HP, regeneration and ticks: the player and
// every monster stand still, so no monster can wake (detection depends on positions only)
// and none acts, the view, memory, frontier list and sightings are already current, and no
// random number is drawn. The loop keeps what changes, in the order the turn and the REST
// loop change it. It returns true once HP is full (the REST ends), false before the turn
// that reaches the deadline, which the caller runs as a whole turn (it ends the episode
// and resets the world).
__device__ __forceinline__ bool rest_quiet(LCtx &c, int limit, POut &o, int &elapsed, float &total, float &discounted,
                                           float &factor) {
    Ctx &x = c.x;
    const D1Config *cf = x.c;
    while (x.ticks + 1 < limit) {
        x.regen += cf->regen;
        while (x.regen >= 100) { x.hp = imin(cf->hp, x.hp + 1); x.regen -= 100; }
        x.ticks++;
        elapsed++;
        total += o.reward;
        discounted += factor * o.reward;
        factor *= 1.f;
        o.hp = imax(0, x.hp);
        o.ticks = x.ticks;
        if (x.hp >= cf->hp) return true;
    }
    return false;
}

// Joint action (learn.cu:853-875): MOVE 0-7, ATTACK 8-15, WAIT 16, REST 17, DESCEND 18.
template <int CLUMP>
__device__ __forceinline__ void transition_learn(LCtx &c, int action, int limit, float *out) {
    Ctx &x = c.x;
    const D1Config *cf = x.c;
    const int decisions = x.decisions + 1, initial_hp = x.hp;
    int elapsed = 0, interrupted = 0, invalid = 0;
    float total = 0.f, discounted = 0.f, factor = 1.f;
    POut o;
    for (int guard = 0; guard < (1 << 16); guard++) {
        int d = 8;
        if (action >= 0 && action < 16) {
            int dir = action % 8, p = nbr(x.player, dir);
            bool enemy = p >= 0 && in_view(x, p) && bit(x.sm->occ, p);
            bool valid = action < 8 ? p >= 0 && (!bit(x.sm->viewed, p) || bit(x.sm->floor, p)) && !enemy : enemy;
            if (valid) d = dir; else invalid = 1;
        } else if (action == 17) invalid = x.hp >= cf->hp || visible_awake(x) || cf->regen <= 0;
        else if (action == 18) { if (stair_index(x) > 0) d = 18; else invalid = 1; }
        else if (action != 16) invalid = 1;
        primitive_learn<CLUMP>(c, d, limit, o);
        elapsed++;
        total += o.reward;
        discounted += factor * o.reward;
        factor *= 1.f;
        if (o.done || invalid || action != 17) break;
        interrupted = o.saw_awake;
        if (interrupted || x.hp >= cf->hp) break;
        if (!ballot(lane_alive(c) && x.mawake) && rest_quiet(c, limit, o, elapsed, total, discounted, factor)) break;
    }
    if (!o.done) x.decisions = decisions;
    if (!out) return;
    float v = 0.f;
    switch (x.lane) {   // one outcome field per lane (learn.cu:801-822, 869-874)
    case 0: v = total; break;
    case 1: v = (float)o.done; break;
    case 2: v = (float)o.clear; break;
    case 3: v = (float)o.killed; break;
    case 4: v = (float)o.hp; break;
    case 5: v = (float)o.ticks; break;
    case 6: v = (float)o.death; break;
    case 7: v = (float)o.timeout; break;
    case 8: v = (float)o.enc; break;
    case 9: v = (float)o.alive_unenc; break;
    case 10: v = (float)o.alive_enc; break;
    case 11: v = (float)o.floor_seen / (float)o.ncells; break;
    case 12: v = (float)o.vis; break;
    case 13: v = (float)o.floor_seen; break;
    case 26: v = (float)elapsed; break;
    case 33: v = (float)o.saw_enemy; break;
    case 34: v = action == 17 ? 1.f : 0.f; break;
    case 35: v = action == 17 ? (float)elapsed : 0.f; break;
    case 36: v = action == 17 ? (float)(!o.done && x.hp >= cf->hp) : 0.f; break;
    case 37: v = action == 17 ? (float)interrupted : 0.f; break;
    case 38: v = action == 17 ? (float)invalid : 0.f; break;
    case 39: v = action == 17 ? (float)imax(0, o.hp - initial_hp) : 0.f; break;
    case 40: v = discounted; break;
    case 41: v = (float)o.saw_awake; break;
    case 42: v = (float)o.known; break;
    case 43: v = (float)o.first_tick; break;
    case 44: v = (float)o.stair; break;
    default: break;
    }
    if (x.lane < D1L_OUT) out[x.lane] = v;
}

// ---------------------------------------------------------------- observation (learn.cu:480-682)
__device__ __forceinline__ void observe_learn(LCtx &c, float *obs, float *mask) {
    Ctx &x = c.x;
    Smem *sm = x.sm;
    const D1Config *cf = x.c;
    const int px = x.player % W, py = x.player / W;
    const int seen = seen_stairs(x), ks = __popc(seen);
    // frontier pointer and stair cue from one known-floor BFS
    anchors_all(c);
    KB r{-1, -1, -1, -1, -1};
    if (c.nf > 0 || ks > 0) r = known_bfs(c, c.nf > 0, ks > 0 ? seen : 0, false);
    int best = r.alayer >= 0 ? first_hit(c) : -1;
    float f[7] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int fdir = -1;
    if (best >= 0) {
        int unseen = 0, bdx = 0, bdy = 0;
        for (int d = 0; d < 8; d++) {
            int q = nbr(best, d);
            if (q >= 0 && !bit(sm->viewed, q) && ++unseen == 1) { bdx = q % W - best % W; bdy = q / W - best / W; }
        }
        f[0] = 1.f;
        f[1] = (best % W - px) / (float)W;
        f[2] = (best / W - py) / (float)H;
        f[3] = r.alayer / (float)(W + H);
        f[4] = unseen / 8.f;
        f[5] = (float)bdx;
        f[6] = (float)bdy;
        fdir = route_first_step(c, best, r.alayer);
    }
    int sD = 65535, target = ks ? nearest_stair(x, seen, r, sD) : -1;
    int sdir = target >= 0 ? route_first_step(c, target, sD) : -1;
    const bool on_stair = stair_index(x) > 0;
    const bool rest_ok = x.hp < cf->hp && cf->regen > 0 && !visible_awake(x);
    __syncthreads();
    float *ob = sm->stage;   // overlays the BFS bitmaps, which are no longer needed
    for (int j = x.lane; j < D1L_OBS; j += 64) ob[j] = 0.f;
    __syncthreads();
    for (int w = x.lane; w < 225; w += 64) {
        int dx = w % 15 - 7, dy = w / 15 - 7, xx = px + dx, yy = py + dy;
        if (!inb(xx, yy)) continue;
        bool vw = bit_at(sm->viewed, xx, yy);
        ob[w] = vw ? (bit_at(sm->floor, xx, yy) ? 1.f : -1.f) : 0.f;
        ob[O_VISIBLE + w] = vis_rel(x, dx, dy) ? 1.f : 0.f;
    }
    if (lane_alive(c) && in_view(x, x.mpos)) {
        int dx = x.mpos % W - px, dy = x.mpos / W - py;
        ob[O_ENEMY_HP + (dy + 7) * 15 + dx + 7] = x.mhp / 16.f;
        float *rec = ob + O_RECORDS + c.mslot * 5;
        rec[0] = dx / 80.f;
        rec[1] = dy / 70.f;
        rec[2] = x.mhp / 16.f;
        rec[3] = (x.lane % 6) / 5.f;
        rec[4] = 1.f;
        ob[O_SLEEP + c.mslot] = x.mawake ? -1.f : 1.f;
    }
    {   // ring of radius 8, indexed as learn.cu:535-541
        int j = x.lane, rx, ry;
        if (j < 17) { ry = -8; rx = j - 8; }
        else if (j < 34) { ry = 8; rx = j - 25; }
        else if (j < 49) { rx = -8; ry = j - 41; }
        else { rx = 8; ry = j - 56; }
        int xx = px + rx, yy = py + ry;
        if (inb(xx, yy) && bit_at(sm->viewed, xx, yy)) ob[O_RING + j] = bit_at(sm->floor, xx, yy) ? 1.f : -1.f;
    }
    if (x.lane == 0) {
        ob[O_PLAYER] = x.hp / (float)cf->hp;
        ob[O_PLAYER + 1] = x.ticks / 2048.f;
        ob[O_PLAYER + 2] = px / 80.f;
        ob[O_PLAYER + 3] = py / 70.f;
        ob[O_PROGRESS] = x.floor_seen / 1024.f;
        ob[O_STAIR] = ks / 3.f;
        ob[O_STAIR + 15] = on_stair ? 1.f : 0.f;
        if (target >= 0) {
            ob[O_STAIR + 1] = 1.f;
            ob[O_STAIR + 2] = (target % W - px) / (float)W;
            ob[O_STAIR + 3] = (target / W - py) / (float)H;
            ob[O_STAIR + 4] = sD / (float)(W + H);
            if (sdir >= 0) {
                int q = nbr(x.player, sdir);
                ob[O_STAIR + 5] = (float)(q % W - px);
                ob[O_STAIR + 6] = (float)(q / W - py);
                ob[O_STAIR + 7 + sdir] = 1.f;
            }
        }
        if (fdir >= 0) ob[O_FRONTIER + 7 + fdir] = 1.f;
    }
    if (x.lane < 7) {
        float v = f[0];
        for (int k = 1; k < 7; k++) v = x.lane == k ? f[k] : v;
        ob[O_FRONTIER + x.lane] = v;
    }
    __syncthreads();
    if (obs)
        for (int j = x.lane; j < D1L_OBS; j += 64) obs[j] = ob[j];
    if (mask && x.lane < D1L_ACTIONS) {
        float v;
        if (x.lane < 16) {
            int p = nbr(x.player, x.lane & 7);
            bool enemy = p >= 0 && in_view(x, p) && bit(sm->occ, p);
            v = x.lane < 8 ? (float)(p >= 0 && (!bit(sm->viewed, p) || bit(sm->floor, p)) && !enemy) : (float)enemy;
        } else v = x.lane == 16 ? 1.f : x.lane == 17 ? (float)rest_ok : (float)on_stair;
        mask[x.lane] = v;
    }
    __syncthreads();
}

// ---------------------------------------------------------------- controller (learn.cu:452-479,876-888)
__device__ __forceinline__ int heuristic_learn(LCtx &c) {
    Ctx &x = c.x;
    Smem *sm = x.sm;
    const D1Config *cf = x.c;
    if (stair_index(x) > 0) return 18;
    // weakest visible adjacent enemy, first direction on ties
    bool adj = lane_alive(c) && cheb(x.mpos, x.player) == 1 && in_view(x, x.mpos);
    int dir = 0;
    if (adj)
        for (int d = 0; d < 8; d++) dir = nbr(x.player, d) == x.mpos ? d : dir;
    int akey = wave_min(adj ? x.mhp * 8 + dir : INF);
    if (akey != INF) return 8 + (akey & 7);
    const bool vawake = visible_awake(x);
    if (x.hp < cf->hp && cf->regen > 0 && !vawake) return 17;
    if (vawake) return 16;
    const int seen = seen_stairs(x), ks = __popc(seen);
    const bool venemy = visible_enemy(c);
    // one BFS serves the stair route, the engage target and the explore target
    anchors_all(c);
    const bool want_anchor = !venemy && c.nf > 0;
    KB r{-1, -1, -1, -1, -1};
    if (ks || venemy || want_anchor) r = known_bfs(c, want_anchor, ks ? seen : 0, venemy);
    if (ks) {
        int sD = 65535, target = nearest_stair(x, seen, r, sD);
        int d = target >= 0 ? route_first_step(c, target, sD) : -1;
        if (d >= 0) {
            int p = nbr(x.player, d);
            if (!(bit(sm->occ, p) && in_view(x, p))) return d;
        }
    }
    if (venemy) {   // engage: nearest visible enemy by known distance, slot order on ties
        bool cand = lane_alive(c) && in_view(x, x.mpos) && r.mlayer >= 0;
        int ekey = wave_min(cand ? r.mlayer * 64 + c.mslot : INF);
        if (ekey != INF) {
            uint64_t who = ballot(cand && r.mlayer * 64 + c.mslot == ekey);
            int target = lane_val(x.mpos, __ffsll((unsigned long long)who) - 1);
            int d = route_first_step(c, target, ekey >> 6);
            if (d >= 0) {
                int q = nbr(x.player, d);
                if (q >= 0 && !(bit(sm->occ, q) && in_view(x, q))) return d;
            }
        }
        return 16;   // explore_step declines while an enemy is visible
    }
    int best = r.alayer >= 0 ? first_hit(c) : -1;
    if (best < 0) return 16;
    if (best != x.player) {
        int d = route_first_step(c, best, r.alayer);
        return d >= 0 ? d : 16;
    }
    uint64_t un = ballot(x.lane < 8 && nbr(x.player, x.lane) >= 0 && !bit(sm->viewed, nbr(x.player, x.lane)));
    return un ? __ffsll((unsigned long long)un) - 1 : 16;
}

// ---------------------------------------------------------------- load / store
__device__ __forceinline__ void load_learn(LCtx &c, const uint8_t *row) {
    Ctx &x = c.x;
    const LHdr h = *(const LHdr *)row;
    x.g.pcg_load(h.rng_state, h.rng_inc);
    c.enc = h.encountered;
    x.ticks = h.ticks; x.killed = h.killed; x.decisions = h.decisions; x.floor_seen = h.floor_seen;
    x.episode = h.episode; x.first_stair_tick = h.first_stair_tick;
    x.player = h.player; x.hp = h.hp; x.regen = h.regen; x.blocks = h.blocks;
    c.map_id = h.map_id; c.next_slot = h.next_slot; c.nf = imin(imax((int)h.frontier_count, 0), N);
    x.stairs = pack_stairs(h.stairs[0], h.stairs[1], h.stairs[2]);
    c.clumped = h.clumped; c.error = h.error;
    // a row that is not this library's (or a map index beyond the tables) is flagged
    // and clamped so that no table access leaves its bounds
    if (c.map_id < 0 || c.map_id >= c.t->n_maps) { c.error = 1; c.map_id = 0; }
    if (x.player < 0 || x.player >= N) { c.error = 1; x.player = 0; }
    c.los = c.t->los + (size_t)c.map_id * N * 10;
    LMon m{-1, 0, -30000, 0, -1};
    if (x.lane < REQ) m = ((const LMon *)(row + OFF_MON))[x.lane];
    if (m.hp > 0 && (m.pos < 0 || m.pos >= N)) { m.hp = 0; m.energy = -30000; }
    if (m.slot >= LE) m.slot = -1;
    x.mpos = m.pos; x.mhp = m.hp; x.menergy = m.energy; x.mawake = m.awake; x.mkind = x.lane % 6; c.mslot = m.slot;
    const uint32_t *vg = (const uint32_t *)(row + OFF_VIEWED), *fg = (const uint32_t *)(row + OFF_FLOOR);
    for (int w = x.lane; w < ROWS_WORDS; w += 64) { x.sm->viewed[w] = vg[w]; x.sm->floor[w] = fg[w]; x.sm->occ[w] = 0; }
    c.lst = (uint16_t *)(row + OFF_LIST);
    __syncthreads();
    if (lane_alive(c)) occ_set_lane(x, x.mpos);
    __syncthreads();
}
__device__ __forceinline__ void store_learn(LCtx &c, uint8_t *row) {
    Ctx &x = c.x;
    if (x.lane == 0) {
        LHdr h{};
        h.rng_state = x.g.pcg_state(); h.rng_inc = x.g.inc; h.encountered = c.enc;
        h.ticks = x.ticks; h.killed = x.killed; h.decisions = x.decisions; h.floor_seen = x.floor_seen;
        h.episode = x.episode; h.first_stair_tick = x.first_stair_tick;
        h.player = (int16_t)x.player; h.hp = (int16_t)x.hp; h.regen = (int16_t)x.regen; h.blocks = (int16_t)x.blocks;
        h.map_id = (int16_t)c.map_id; h.next_slot = (int16_t)c.next_slot; h.frontier_count = (int16_t)c.nf;
        h.stairs[0] = (int16_t)stair_at(x, 0); h.stairs[1] = (int16_t)stair_at(x, 1); h.stairs[2] = (int16_t)stair_at(x, 2);
        h.clumped = (uint8_t)c.clumped; h.error = (uint8_t)c.error;
        *(LHdr *)row = h;
    }
    if (x.lane < REQ) {
        LMon m;
        m.pos = (int16_t)x.mpos; m.hp = (int16_t)x.mhp; m.energy = (int16_t)x.menergy;
        m.awake = (uint8_t)x.mawake; m.slot = (int8_t)c.mslot;
        ((LMon *)(row + OFF_MON))[x.lane] = m;
    }
    uint32_t *vg = (uint32_t *)(row + OFF_VIEWED);
    for (int w = x.lane; w < ROWS_WORDS; w += 64) vg[w] = x.sm->viewed[w];
}
__device__ __forceinline__ void store_floor(LCtx &c, uint8_t *row) {
    uint32_t *fg = (uint32_t *)(row + OFF_FLOOR);
    for (int w = c.x.lane; w < ROWS_WORDS; w += 64) fg[w] = c.x.sm->floor[w];
}
__device__ __forceinline__ void setup(LCtx &c, LSmem *L, const D1Config *cfg, const D1LTables *t) {
    c.L = L; c.t = t;
    c.x.sm = &L->s; c.x.c = cfg; c.x.rays = nullptr; c.x.nslots = 0; c.x.lane = lane_id();
    c.x.t = 0; c.x.env_id = 0; c.x.ncells = 0;
    set_view(c.x, 0, 0, 0, 0);
    c.clumped = 0; c.error = 0;
}

// ---------------------------------------------------------------- kernels
template <int CLUMP>
__global__ __launch_bounds__(64) void k_learn_init(uint8_t *state, int n, D1Config cfg, D1LTables t, uint64_t seed,
                                                   float *obs, float *mask) {
    __shared__ LSmem L;
    int env = blockIdx.x;
    if (env >= n) return;
    uint8_t *row = state + (size_t)env * ROW_BYTES;
    LCtx c;
    D1LTables first = t;
    if (first.map_filter == -2) first.map_filter = env % first.n_maps;
    setup(c, &L, &cfg, &first);
    c.lst = (uint16_t *)(row + OFF_LIST);
    c.x.g.pcg_seed(mix64(seed + (uint64_t)env), (uint64_t)env + 1);
    c.x.episode = 0; c.x.decisions = 0;
    reset_learn<CLUMP>(c);
    c.t = &t;
    store_learn(c, row);
    store_floor(c, row);
    observe_learn(c, obs ? obs + (size_t)env * D1L_OBS : nullptr, mask ? mask + (size_t)env * D1L_ACTIONS : nullptr);
}
template <int CLUMP>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(4))) void k_learn_step(uint8_t *state, int n, D1Config cfg, D1LTables t,
                                                   const int64_t *actions, int limit, float *obs, float *mask,
                                                   float *out, const bool *active) {
    __shared__ LSmem L;
    int env = blockIdx.x;
    if (env >= n) return;
    if (active && !active[env]) return;
    uint8_t *row = state + (size_t)env * ROW_BYTES;
    LCtx c;
    setup(c, &L, &cfg, &t);
    load_learn(c, row);
    const int episode = c.x.episode;
    const int action = (int)actions[env];   // the low 32 bits, as the reference's int parameter
    view_los(c);
    transition_learn<CLUMP>(c, action, limit, out ? out + (size_t)env * D1L_OUT : nullptr);
    store_learn(c, row);
    if (c.x.episode != episode) store_floor(c, row);   // a reset may have changed the map
    observe_learn(c, obs ? obs + (size_t)env * D1L_OBS : nullptr, mask ? mask + (size_t)env * D1L_ACTIONS : nullptr);
}
__global__ __launch_bounds__(64) void k_learn_heuristic(const uint8_t *state, int n, D1Config cfg, D1LTables t,
                                                        int64_t *actions) {
    __shared__ LSmem L;
    int env = blockIdx.x;
    if (env >= n) return;
    LCtx c;
    setup(c, &L, &cfg, &t);
    load_learn(c, state + (size_t)env * ROW_BYTES);
    view_los(c);
    int a = heuristic_learn(c);
    if (c.x.lane == 0) actions[env] = a;
}

int validate(int n, const D1LConfig *c, const D1LTables *t) {
    if (n < 0 || !c || !t || !t->floor || !t->cells || !t->map_ncells || !t->los) return D1L_E_ARG;
    if (t->n_maps < 1 || t->map_filter < -2 || t->map_filter >= t->n_maps) return D1L_E_ARG;
    if (c->count != REQ) return D1L_E_CONFIG;
    if (c->hp < 1 || c->hp > 30000 || c->ac100 < 0 || c->ev100 < 0 || c->sh100 < 0 || c->regen < 0) return D1L_E_CONFIG;
    for (int k = 0; k < 2; k++) if (c->gdr[k] < 0) return D1L_E_CONFIG;
    for (int k = 0; k < 6; k++)
        if (c->kinds[k].speed < 0 || c->kinds[k].speed > 20 || c->kinds[k].damage < 0 || c->kinds[k].tohit < 0 ||
            c->kinds[k].bypass < 0)
            return D1L_E_CONFIG;
    return 0;
}
// The shared device core reads the simulator fields of D1Config.
D1Config core_config(const D1LConfig *c) {
    D1Config d{};
    d.count = c->count; d.hp = c->hp; d.ac100 = c->ac100; d.ev100 = c->ev100; d.sh100 = c->sh100;
    d.shield_limit = c->shield_limit; d.regen = c->regen; d.repair = c->repair;
    d.gdr[0] = c->gdr[0]; d.gdr[1] = c->gdr[1];
    for (int k = 0; k < 6; k++)
        d.kinds[k] = D1Kind{c->kinds[k].speed, c->kinds[k].damage, c->kinds[k].tohit, c->kinds[k].bypass};
    d.limit = 2048; d.wake_los = 1; d.stairs = 3;
    return d;
}

}  // namespace learn
}  // namespace d1

extern "C" {
float learn_turn_cost(void) { return d1::learn::TURN_COST; }
float learn_return_gamma(void) { return 1.f; }
int learn_state_bytes(void) { return d1::learn::ROW_BYTES; }
int learn_obs_size(void) { return D1L_OBS; }
int learn_action_size(void) { return D1L_ACTIONS; }
int learn_out_size(void) { return D1L_OUT; }
int learn_config_bytes(void) { return (int)sizeof(D1LConfig); }

int learn_init(void *state, int n, const D1LConfig *cfg, const D1LTables *tab, uint64_t seed, float *obs,
               float *mask, void *stream, int gpu) {
    int e = d1::learn::validate(n, cfg, tab);
    if (e) return e;
    if (!gpu) return D1L_E_HOST;
    if (!state) return D1L_E_ARG;
    if (n == 0) return 0;
    hipLaunchKernelGGL(d1::learn::k_learn_init<D1_CLUMP_MODE>, dim3(n), dim3(64), 0, (hipStream_t)stream,
                       (uint8_t *)state, n, d1::learn::core_config(cfg), *tab, seed, obs, mask);
    return (int)hipGetLastError();
}
int learn_step_active(void *state, int n, const D1LConfig *cfg, const D1LTables *tab, const int64_t *actions,
                      int limit, float *obs, float *mask, float *out, const bool *active, void *stream, int gpu) {
    int e = d1::learn::validate(n, cfg, tab);
    if (e) return e;
    if (!gpu) return D1L_E_HOST;
    if (!state || !actions || limit < 1) return D1L_E_ARG;
    if (n == 0) return 0;
    hipLaunchKernelGGL(d1::learn::k_learn_step<D1_CLUMP_MODE>, dim3(n), dim3(64), 0, (hipStream_t)stream,
                       (uint8_t *)state, n, d1::learn::core_config(cfg), *tab, actions, limit, obs, mask, out, active);
    return (int)hipGetLastError();
}
int learn_step(void *state, int n, const D1LConfig *cfg, const D1LTables *tab, const int64_t *actions, int limit,
               float *obs, float *mask, float *out, void *stream, int gpu) {
    return learn_step_active(state, n, cfg, tab, actions, limit, obs, mask, out, nullptr, stream, gpu);
}
int learn_heuristic(void *state, int n, const D1LConfig *cfg, const D1LTables *tab, int64_t *actions, void *stream,
                    int gpu) {
    int e = d1::learn::validate(n, cfg, tab);
    if (e) return e;
    if (!gpu) return D1L_E_HOST;
    if (!state || !actions) return D1L_E_ARG;
    if (n == 0) return 0;
    hipLaunchKernelGGL(d1::learn::k_learn_heuristic, dim3(n), dim3(64), 0, (hipStream_t)stream,
                       (const uint8_t *)state, n, d1::learn::core_config(cfg), *tab, actions);
    return (int)hipGetLastError();
}
}
