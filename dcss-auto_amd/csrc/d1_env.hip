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

#include "d1_core.h"

namespace d1 {

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

// the player's view (4 x u64 quadrant sets) is kept beside the header: it only changes
// when the player moves, so a step that does not move needs no LOS scan and no reveal
constexpr int OFF_VIEW = 64, OFF_MON = 96;
__host__ __device__ constexpr int off_viewed(int m) { return OFF_MON + 8 * m; }
__host__ __device__ constexpr int off_floor(int m) { return off_viewed(m) + ROWS_WORDS * 4; }
__host__ __device__ constexpr int off_cells(int m) { return off_floor(m) + ROWS_WORDS * 4; }
// Layouts with more than 8 monsters also keep the distance-field memo: dword 0 the player
// cell it was computed for (-1: none), dword 1 its last layer (bit 31: the reach bitmap
// equals the floor bitmap and is not stored), dwords 2-33 the monsters' absolute layers
// (int16 each, 32767 = unknown), dwords 34-49 the monsters' stuck-cache radii (uint8 each,
// 0 = none; Ctx::mrad), then the reach, lay0 and lay1 bitmaps.
constexpr int FC_RAD = 34, FC_HEAD = 50, FC_DWORDS = FC_HEAD + 3 * ROWS_WORDS;
__host__ __device__ constexpr bool has_fcache(int m) { return m > 8; }
__host__ __device__ constexpr int off_fcache(int m) { return off_cells(m) + ROWS_WORDS * 4; }
__host__ __device__ constexpr int state_bytes(int m) {
    return (off_fcache(m) + (has_fcache(m) ? FC_DWORDS * 4 : 0) + 63) / 64 * 64;
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
    x.vlo = 0, x.vhi = H - 1;
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
    x.ftag = -1;   // a new player cell and new monster cells: the memo no longer applies
    x.fld = -1;    // and the reach bitmap held the stairs' eligible cells
    x.mrad = 0;    // nor does any stuck answer
}

// ---------------------------------------------------------------- distance-field memo
// The distance field is a function of the level and the player's cell only. The crowded
// layouts keep a complete field (BFS to exhaustion, every living monster's layer recorded)
// in the state row and reuse it while the player stays on that cell; monster moves keep
// their layers exact (a move is to a reached neighbour, one of -1/0/+1 away). A step whose
// player stands still then reads 1,680 bytes (2,520 where the level is not connected)
// instead of running the whole BFS.
__device__ __forceinline__ void field_memo(Ctx &x) {
    if (x.fld == x.player) return;   // LDS holds it already (a REST repeat)
    Smem *sm = x.sm;
    uint32_t *fc = x.fcache;
    if (x.ftag == x.player) {
        if (x.rfloor) {
            for (int w = x.lane; w < ROWS_WORDS; w += 64) sm->reach[w] = sm->floor[w];
        } else {
            for (int w = x.lane; w < ROWS_WORDS; w += 64) sm->reach[w] = fc[FC_HEAD + w];
        }
        for (int w = x.lane; w < ROWS_WORDS; w += 64) {
            sm->lay0[w] = fc[FC_HEAD + ROWS_WORDS + w];
            sm->lay1[w] = fc[FC_HEAD + 2 * ROWS_WORDS + w];
            sm->front[w] = 0;   // the repair search's queued marks start clear, as after bfs()
        }
        __syncthreads();
    } else {
        const uint64_t living = ballot(x.lane < x.c->count && x.mhp > 0);
        bfs(x, living, BIG);
        // On a connected level the complete field reaches every floor cell: the reach plane
        // is then not stored, and a reload takes the floor bitmap for it (840 bytes less each
        // way).
        bool same = true;
        for (int w = x.lane; w < ROWS_WORDS; w += 64) same = same && sm->reach[w] == sm->floor[w];
        x.rfloor = !ballot(!same);
        for (int w = x.lane; w < ROWS_WORDS; w += 64) {
            if (!x.rfloor) fc[FC_HEAD + w] = sm->reach[w];
            fc[FC_HEAD + ROWS_WORDS + w] = sm->lay0[w];
            fc[FC_HEAD + 2 * ROWS_WORDS + w] = sm->lay1[w];
        }
        x.ftag = x.player;
    }
    x.fld = x.player;
}

// ---------------------------------------------------------------- one physical turn
// gpu-d1/branches/d1-stairs-v2/src/learn.cu:684-827 with the v1 kill-all clear
// (gpu-d1/src/learn.cu:549) as a switch. d: 0-7 move/bump, 8 wait, 18 descend.
// Returns done; out8 = reward, done, clear, killed, hp, ticks, death, timeout.
// `saw` (an awake monster was in view during the turn) is computed only when want_saw: REST
// repeats read it, every other action ignores it.
__device__ __forceinline__ bool primitive(Ctx &x, int d, float *out8, bool &saw, bool want_saw, const uint32_t *cells_g) {
    const D1Config *c = x.c;
    Smem *sm = x.sm;
    int milli = c->step_milli;
    bool moved = false;
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
                        if (x.stuck_cache) stuck_touch(x, p, p);   // its cell frees
                        occ_set(x, p, false);
                        x.killed++;
                        milli += c->kill_milli;
                    } else if (x.lane == id) x.mhp = nh;
                }
            } else {
                x.player = p;
                moved = true;
                x.mrad = 0;   // a new distance field: no stuck answer stands
            }
        }
    }
    if (moved) milli += c->explore_milli * reveal(x);   // an unmoved view reveals nothing new
    saw = want_saw && visible_awake(x);
    bool clear = (d == 18 && stair_index(x) > 0 && x.hp > 0) || (c->clear_on_kill_all && x.killed == c->count);
    if (!clear) {
        bool mine = x.lane < c->count;
        uint64_t cand = ballot(mine && x.mhp > 0 && !x.mawake && cheb_u(x.mpos, x.player) <= 6);
        while (cand) {
            int i = __ffsll((unsigned long long)cand) - 1;
            cand &= cand - 1;
            int pos = lane_val(x.mpos, i);
            if (detects(x, pos) && x.lane == i) { x.mawake = 1; x.menergy = 70; }
        }
        if (mine && x.mhp > 0 && !x.mawake) x.menergy = -30000;
        if (mine && x.mhp > 0) x.menergy += kind_speed(c, x.mkind);
        x.menergy = (int16_t)x.menergy;
        uint64_t movers = ballot(mine && x.mhp > 0 && x.mawake && x.menergy >= 80 && cheb_u(x.mpos, x.player) > 1);
        if (movers) {
            if (x.fcache) field_memo(x);
            else {
                int maxspeed = 0;
                for (int k = 0; k < 6; k++) maxspeed = imax(maxspeed, c->kinds[k].speed);
                bfs(x, movers, imax(2, (maxspeed + 9) / 10));
            }
        }
        // a ballot ends the loop when no monster can act (most turns), before any reduction
        while (x.hp > 0 && ballot(mine && x.menergy >= 80)) {
            // The lane id made opaque per act: the lane-derived addresses and masks of the
            // monster rules are then recomputed in each act instead of being held from the
            // world's start through the whole loop, where the crowded build (80 VGPRs at 6
            // waves per SIMD) spilled them to scratch and both builds spilled their lane masks
            // from SGPRs to VGPR lanes (k_step_crowd 2.30 -> 2.16 ms at C5, k_step 0.158 ->
            // 0.152 ms at C3).
            {
                int l = lane_id();
                asm volatile("" : "+v"(l));
                x.lane = l;
            }
            const int key = wave_max(mine && x.menergy >= 80 ? x.menergy * 128 + 127 - x.lane : -1);
            int id = 127 - (key & 127);
            act(x, id);
            if (want_saw && !saw && in_view(x, lane_val(x.mpos, id))) saw = true;
        }
    }
    x.ticks++;
    // A stair becomes known only through a reveal: this turn's (a move) or the reset's, which
    // runs after the previous turn's check (the first turn of an episode, ticks == 1).
    if (x.first_stair_tick < 0 && (moved || x.ticks == 1) && known_stairs(x) > 0) x.first_stair_tick = x.ticks;
    bool death = x.hp <= 0, timeout = !clear && !death && x.ticks >= c->limit;
    if (clear) milli += c->clear_milli;
    if (death) milli -= c->death_milli;
    float reward = 0.001f * (float)milli;
    reward -= c->turn_cost;
    saw = saw || (want_saw && visible_awake(x));
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
            bool enemy = p >= 0 && in_view(x, p) && bit(x.sm->occ, p);
            bool valid = action < 8 ? p >= 0 && (!bit(x.sm->viewed, p) || bit(x.sm->floor, p)) && !enemy : enemy;
            if (valid) d = dir; else invalid = true;
        } else if (action == 17) invalid = x.hp >= c->hp || visible_awake(x) || c->regen <= 0;
        else if (action == 18) { if (stair_index(x) > 0) d = 18; else invalid = true; }
        else if (action != 16) invalid = true;
        bool saw = false;
        bool done = primitive(x, d, out8, saw, action == 17, cells_g);
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
//
// Lanes 0..14 build their window row (dy = lane - 7) as 15-bit strips (bit k = column
// px - 7 + k): wall | viewed-floor << 16 in w0, visible | frontier << 16 in w1, staged in
// LDS. Each row is worked on as one 32-column window of the bitmaps (not their three
// 32-bit words). A cell lane reads its row's pair and assembles its 8 bytes from single
// bits; the lanes of the living monsters and of the known stairs then write their bytes
// over their cells (loops over the window's monsters and stairs, each testing the four
// cells of every lane, cost more than the rest of the observation at 8 monsters).
// 32 columns of bitmap row y from column s (bit j = column s + j), s = 32k + sh with k the
// uniform word index (-1..2): two adjacent words and one funnel shift. Left of the map (k = -1)
// the low word is zero; right of it the high word is the next row's first. Bits of columns
// outside 0..W-1 are arbitrary: every use masks them.
__device__ __forceinline__ uint32_t win32(const uint32_t *bm, int y, int k, uint32_t sh) {
    const uint32_t *w = bm + y * RW + imax(k, 0);
    const uint32_t a = w[0], b = w[1];
    return __builtin_amdgcn_alignbit(k < 0 ? a : b, k < 0 ? 0u : a, sh);
}
__device__ __forceinline__ void write_obs(Ctx &x, uint8_t *o) {
    Smem *sm = x.sm;
    const int px = x.player % W, py = x.player / W;
    uint32_t w0 = 0x7FFFu, w1 = 0;   // rows outside the map: all wall
    {
        const int dy = x.lane - 7, y = py + dy;
        if (x.lane < 15 && y >= 0 && y < H) {
            // one 32-column window per row, s = px - 8: the window's columns px-7 .. px+7 are
            // its bits 1..15, and bits 0 and 16 the columns the frontier's dilation reads
            const int s = px - 8, k = s >> 5;
            const uint32_t sh = (uint32_t)s & 31u;
            const uint32_t ibx = ((2u << imin(31, W - 1 - s)) - 1u) & ~((1u << imax(0, -s)) - 1u);   // map columns
            const uint32_t v0 = win32(sm->viewed, y, k, sh), f0 = win32(sm->floor, y, k, sh);
            const uint32_t vm = y > 0 ? win32(sm->viewed, y - 1, k, sh) : ~0u;
            const uint32_t vp = y < H - 1 ? win32(sm->viewed, y + 1, k, sh) : ~0u;
            const uint32_t u = ~(vm & v0 & vp) & ibx;   // unviewed map cells in rows y-1 .. y+1
            const uint32_t ud = u | (u << 1) | (u >> 1);
            const uint32_t ib = (ibx >> 1) & 0x7FFFu;
            const int ay = iabs(dy);
            uint32_t R = 0, L = 0;
            if (dy >= 0) { R |= (uint32_t)(view_q(x, 0) >> (8 * ay)) & 0xFFu; L |= (uint32_t)(view_q(x, 1) >> (8 * ay)) & 0xFFu; }
            if (dy <= 0) { R |= (uint32_t)(view_q(x, 3) >> (8 * ay)) & 0xFFu; L |= (uint32_t)(view_q(x, 2) >> (8 * ay)) & 0xFFu; }
            const uint32_t vis = ((__builtin_bitreverse32(L) >> 24) | (R << 7)) & ib;
            w0 = (((~ibx | (v0 & ~f0)) >> 1) & 0x7FFFu) | (((v0 & f0 & ibx) >> 1) & 0x7FFFu) << 16;
            w1 = vis | (((v0 & f0 & ud & ibx) >> 1) & 0x7FFFu) << 16;
        }
    }
    // The row pairs go to LDS; a cell lane reads its row's pair (one LDS read a cell where two
    // cross-lane shuffles were) and assembles its 8 bytes with two byte permutes.
    if (x.lane < 15) { sm->orow[2 * x.lane] = w0; sm->orow[2 * x.lane + 1] = w1; }
    __syncthreads();
    const uint32_t php8 = (uint32_t)imin(imax(x.hp, 0), 255) << 8;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t cidx = 64u * c + (uint32_t)x.lane;
        if (cidx >= 225u) continue;
        const uint32_t r = (cidx * 4370u) >> 16, k = cidx - 15u * r;   // cidx / 15, exact below 256
        const uint32_t a = (sm->orow[2 * r] >> k) & 0x10001u, b = (sm->orow[2 * r + 1] >> k) & 0x10001u;
        // bytes 0-3 wall, viewed floor, visible, 0 (a's bytes 0 and 2, b's byte 0);
        // bytes 4-7 0, player HP, 0, frontier (b's byte 2)
        const uint32_t lo = __builtin_amdgcn_perm(b, a, 0x0c040200u), hi = __builtin_amdgcn_perm(b, php8, 0x060c010cu);
        *(uint2 *)(o + cidx * 8) = make_uint2(lo, hi);
    }
    // The cells' few other bytes are written over them by the lanes that own the facts. One
    // wave's memory operations take effect in program order, so a wavefront-scope fence (a
    // compiler barrier) is all the ordering these second stores need.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    // a living monster on a visible window cell: kind + 1 and HP (living monsters hold
    // distinct cells)
    if (x.lane < x.c->count && x.mhp > 0) {
        const int dx = x.mpos % W - px, dy = x.mpos / W - py;
        if (iabs(dx) <= 7 && iabs(dy) <= 7 && ((sm->orow[2 * (dy + 7) + 1] >> (dx + 7)) & 1u)) {
            uint8_t *q = o + ((dy + 7) * 15 + dx + 7) * 8;
            q[3] = (uint8_t)(x.mkind + 1);
            q[4] = (uint8_t)imin(x.mhp, 255);
        }
    }
    // a known stair on a viewed floor window cell (lane k: stair k)
    if (x.lane < 3) {
        const int sp = (int16_t)(uint16_t)(x.stairs >> (16 * x.lane)), dx = sp % W - px, dy = sp / W - py;
        if (sp >= 0 && iabs(dx) <= 7 && iabs(dy) <= 7 && ((sm->orow[2 * (dy + 7)] >> (dx + 23)) & 1u))
            o[((dy + 7) * 15 + dx + 7) * 8 + 6] = 1;
    }
}
// Sum over canonical words of fmix32(word ^ index*0x9E3779B9) (index map in
// include/d1hip.h's companion spec: scalars 0-14, monsters 100+2i, viewed 1000+3y+j).
__device__ __forceinline__ uint32_t state_hash(Ctx &x) {
    // scalar words are hashed in uniform code and added once (lane 0)
    uint32_t scal = term((uint32_t)x.player, 0) + term((uint32_t)x.hp, 1) + term((uint32_t)x.regen, 2) +
                    term((uint32_t)x.ticks, 3) + term((uint32_t)x.killed, 4) + term((uint32_t)x.decisions, 5) +
                    term((uint32_t)x.floor_seen, 6) + term((uint32_t)x.episode, 7) +
                    term(x.g.mode == 0 ? (uint32_t)x.g.pcg_state() : 0u, 8) + term(x.g.mode == 0 ? (uint32_t)(x.g.pcg_state() >> 32) : 0u, 9) +
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
__device__ __forceinline__ void store_world(Ctx &x, uint8_t *row, int max_m) {
    if (x.lane == 0) {
        Hdr h;
        h.rng_state = x.g.mode == 0 ? x.g.pcg_state() : ((uint64_t)x.g.key1 << 32 | x.g.key0);
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
        ((Mon *)(row + OFF_MON))[x.lane] = m;
    }
    if (x.lane < 4) {
        const uint64_t v = x.lane == 0 ? view_q(x, 0) : x.lane == 1 ? view_q(x, 1) : x.lane == 2 ? view_q(x, 2) : view_q(x, 3);
        ((uint64_t *)(row + OFF_VIEW))[x.lane] = v;
    }
    // the viewed rows this step changed: the reveal bands of the cells the player moved to,
    // every row after a reset, none when the player did not move
    uint32_t *vg = (uint32_t *)(row + off_viewed(max_m));
    for (int w = RW * x.vlo + x.lane; w < RW * (x.vhi + 1); w += 64) vg[w] = x.sm->viewed[w];
    if (has_fcache(max_m)) {   // memo head: its player cell, last layer, the monsters' layers
        uint32_t *fc = (uint32_t *)(row + off_fcache(max_m));
        if (x.lane == 0) { fc[0] = (uint32_t)x.ftag; fc[1] = (uint32_t)x.lastl | (uint32_t)x.rfloor << 31; }
        if (x.lane < max_m) {
            ((int16_t *)(fc + 2))[x.lane] = (int16_t)imin(x.mlay, 32767);
            ((uint8_t *)(fc + FC_RAD))[x.lane] = (uint8_t)imin(x.mrad, 255);
        }
    }
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

// ---------------------------------------------------------------- prefetched load
// A k_step workgroup runs several consecutive worlds; the next world's row is fetched into
// registers while the current one steps, so its HBM latency is off the critical path.
// Lane l holds dword l of header + view (l < 24), its monster (l < max_m) and words
// l + 64i of the viewed and floor rows; every lane holds the action and the active flag.
// Addresses are clamped in bounds (the lanes past a field read a copy of its last element).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));   // register-resident 8-byte piece
struct Pre {
    uint32_t hv;
    u32x2 mon;
    uint32_t vw[4], fl[4];
    uint32_t fh;   // dword lane of the distance-field memo head (crowded layouts)
    int act;   // the action's low 32 bits
    int on;
};
__device__ __forceinline__ void prefetch_world(Pre &pf, const uint8_t *row, int max_m, const int64_t *actions,
                                               const uint8_t *active, int env, int lane) {
    pf.hv = ((const uint32_t *)row)[imin(lane, 23)];
    pf.mon = ((const u32x2 *)(row + OFF_MON))[imin(lane, max_m - 1)];
    const uint32_t *vg = (const uint32_t *)(row + off_viewed(max_m)), *fg = (const uint32_t *)(row + off_floor(max_m));
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int w = imin(lane + 64 * i, ROWS_WORDS - 1);
        pf.vw[i] = vg[w];
        pf.fl[i] = fg[w];
    }
    pf.fh = has_fcache(max_m) ? ((const uint32_t *)(row + off_fcache(max_m)))[imin(lane, FC_HEAD - 1)] : 0u;
    pf.act = ((const int *)actions)[2 * (size_t)env];   // little-endian: the int64's low half
    pf.on = active ? active[env] : 1;
}
// load_world from the prefetched registers; RM is the config's RNG mode (a compile-time
// constant, so a kernel carries one generator's state and code)
template <int RM>
__device__ __forceinline__ void unpack_world(Ctx &x, const Pre &pf, int max_m) {
    auto hw = [&](int k) { return (uint32_t)__builtin_amdgcn_readlane((int)pf.hv, k); };
    x.env_id = hw(4); x.t = hw(5); x.episode = (int)hw(6);
    x.player = (int16_t)(hw(7) & 0xFFFFu); x.hp = (int16_t)(hw(7) >> 16);
    x.regen = (int16_t)(hw(8) & 0xFFFFu); x.ncells = (int16_t)(hw(8) >> 16);
    x.ticks = (int)hw(9); x.killed = (int)hw(10); x.decisions = (int)hw(11); x.floor_seen = (int)hw(12);
    x.stairs = pack_stairs((int16_t)(hw(13) & 0xFFFFu), (int16_t)(hw(13) >> 16), (int16_t)(hw(14) & 0xFFFFu));
    x.blocks = (int16_t)(hw(14) >> 16); x.first_stair_tick = (int)hw(15);
    const uint64_t rs = (uint64_t)hw(1) << 32 | hw(0), ri = (uint64_t)hw(3) << 32 | hw(2);
    if (RM == 0) x.g.pcg_load(rs, ri);
    else x.g.counter(rs, x.env_id, x.t, 0);
    set_view(x, (uint64_t)hw(17) << 32 | hw(16), (uint64_t)hw(19) << 32 | hw(18), (uint64_t)hw(21) << 32 | hw(20),
             (uint64_t)hw(23) << 32 | hw(22));
    if (x.lane < max_m) {
        x.mpos = (int16_t)(pf.mon.x & 0xFFFFu); x.mhp = (int16_t)(pf.mon.x >> 16);
        x.menergy = (int16_t)(pf.mon.y & 0xFFFFu); x.mawake = (pf.mon.y >> 16) & 0xFFu; x.mkind = pf.mon.y >> 24;
    } else {
        x.mpos = -1; x.mhp = 0; x.menergy = -30000; x.mawake = 0; x.mkind = 0;
    }
    x.fld = -1;
    x.vlo = H, x.vhi = -1;   // no viewed row changed yet
    if (has_fcache(max_m)) {
        x.ftag = (int)__builtin_amdgcn_readlane((int)pf.fh, 0);
        const uint32_t h1 = (uint32_t)__builtin_amdgcn_readlane((int)pf.fh, 1);
        x.lastl = (int)(h1 & 0x7FFFFFFFu);
        x.rfloor = h1 >> 31;
        const uint32_t pair = (uint32_t)__shfl((int)pf.fh, 2 + (x.lane >> 1));
        const int ml = (int16_t)(x.lane & 1 ? pair >> 16 : pair & 0xFFFFu);
        x.mlay = ml >= 32767 ? FAR : ml;
        const uint32_t quad = (uint32_t)__shfl((int)pf.fh, FC_RAD + (x.lane >> 2));
        x.mrad = x.lane < max_m ? (int)((quad >> (8 * (x.lane & 3))) & 255u) : 0;
    } else {
        x.ftag = -1;
        x.mrad = 0;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int w = x.lane + 64 * i;
        if (w < ROWS_WORDS) { x.sm->viewed[w] = pf.vw[i]; x.sm->floor[w] = pf.fl[i]; x.sm->occ[w] = 0; }
    }
    __syncthreads();
    if (x.lane < x.c->count && x.mhp > 0)
        atomicOr(&x.sm->occ[(x.mpos / W) * RW + ((x.mpos % W) >> 5)], 1u << ((x.mpos % W) & 31));
    __syncthreads();
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
    x.mlay = FAR; x.lastl = 0;
    reset(x, cg);
    store_world(x, row, max_m);
    if (obs) write_obs(x, obs + (size_t)env * D1_OBS_BYTES);
    if (hash) {   // the digest costs about a tenth of a step: callers that do not ask skip it
        const uint32_t h = state_hash(x);
        if (x.lane == 0) hash[env] = h;
    }
}

// Worlds per k_step workgroup: WPB consecutive worlds (each next world's loads overlap the
// current one's stores and observation, so only a group's first load waits), except the
// last STEP_TAIL worlds, one per workgroup: the workgroups dispatched last then hold one
// world, which shortens the tail in which a few slow worlds (resets, long monster turns)
// run on an otherwise idle chip (k_step 193 -> 187 us at 65,536 worlds). WPB is 4 for the
// <= 8 monster build (0.176 -> 0.171 ms at 65,536 worlds) and 3 for the crowded build
// (C5 k_step: 2 worlds 3.38 ms, 3 worlds 3.35, 4 worlds 3.37). The <= 8 monster build's tail
// is 4,096 worlds: the C3 rollout steps its 65,536 worlds as two ranges of 32,768 on two
// streams, where the other range's kernels fill the idle CUs (rollout 364.7 -> 375.7 M
// decisions/s against a tail of 8,192; 0: 368.2, 2,048: 374.3); the crowded build keeps 8,192
// (C5 k_step 2.063 ms against 2.090 with 4,096).
constexpr int STEP_TAIL = 4096, CROWD_TAIL = 8192, STEP_WPB = 4, CROWD_WPB = 3;
__host__ __device__ inline int step_groups(int n, int wpb, int tail) { return (n - (n < tail ? n : tail)) / wpb; }
__host__ __device__ inline int step_blocks(int n, int wpb, int tail) {
    const int g = step_groups(n, wpb, tail);
    return g + (n - wpb * g);
}
template <int RM, int WPB, bool CROWD>
__device__ __forceinline__ void step_worlds(Smem &sm, uint8_t *state, int n, int max_m, size_t row_bytes,
                                            const D1Config *cfgp, const D1Tables &tab, const int64_t *actions,
                                            uint8_t *obs, float *out, uint32_t *hash, const uint8_t *active) {
    constexpr int TAIL = CROWD ? CROWD_TAIL : STEP_TAIL;
    const int g = step_groups(n, WPB, TAIL), blk = (int)blockIdx.x;   // first < n for every block of step_blocks
    const int first = blk < g ? WPB * blk : WPB * g + (blk - g), last = imin(n, blk < g ? first + WPB : first + 1);
    Ctx x;
    x.sm = &sm; x.c = cfgp; x.rays = tab.ray_slots; x.nslots = tab.nslots; x.lane = lane_id();
    x.view_lds = CROWD;   // the crowded build keeps the player view in LDS
    x.stuck_cache = CROWD;   // and a complete distance field that depends on the player cell alone
    // Each world is loaded when the wave starts it. Fetching the next world's row while the
    // current one stores its state and observation held 12 more registers across those
    // phases: at 4 waves per SIMD it paid (0.176 -> 0.171 ms at C3), but with the lane
    // masks no longer held through the monster loop both builds run more waves per SIMD
    // without it, whose latency hiding does more (C3 k_step 0.152 -> 0.140 ms at 5 waves;
    // in the crowded build the held row had gone to scratch, about 7 KB of traffic a world).
    Pre pf;
    for (int env = first; env < last; env++) {
        // Opaque per world: otherwise every lane-derived constant of the world step is
        // hoisted out of this loop and kept live across it.
        int lane = lane_id();
        asm volatile("" : "+v"(lane));
        x.lane = lane;
        uint8_t *row = state + (size_t)env * row_bytes;
        prefetch_world(pf, row, max_m, actions, active, env, x.lane);
        const int on = __builtin_amdgcn_readfirstlane(pf.on);
        // the int64 action's low 32 bits as a signed int, as the reference's int parameter
        // takes it (gpu-d1/branches/d1-stairs-v2/src/learn.cu:853,904); values outside the
        // action set are invalid actions
        const int action = __builtin_amdgcn_readfirstlane(pf.act);
        if (!on) continue;   // an inactive env keeps its state and all its output rows
        unpack_world<RM>(x, pf, max_m);
        x.fcache = has_fcache(max_m) ? (uint32_t *)(row + off_fcache(max_m)) : nullptr;
        const uint32_t *cg = (const uint32_t *)(row + off_cells(max_m));
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
        if (hash) {   // the digest costs about a tenth of a step: callers that do not ask skip it
            const uint32_t h = state_hash(x);
            if (x.lane == 0) hash[env] = h;
        }
    }
}

// Two builds of the same step. A world with at most 8 monsters spends its time in straight
// issue-bound code (observation, reveal, scalar rules): 4 waves per SIMD without spills. The
// crowded layouts (up to 64 monsters) spend it in serial monster turns whose LDS and
// cross-lane latencies want more waves in flight: 6 waves per SIMD, which costs some
// register spills (measured at 262,144 worlds x 40 monsters: 8.3 -> 7.0 ms per step; at
// 65,536 x 8 the same build is 0.17 -> 0.33 ms, hence two builds). The <= 8 monster build
// reads its configuration from an LDS copy, which keeps the fields out of scalar registers
// (190 -> 104 spilled to VGPR lanes; 0.171 -> 0.168 ms at 65,536 worlds); in the crowded
// build the same copy costs 4.69 -> 5.19 ms, so it reads the kernel argument.
template <int RM>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(5))) void k_step(
    uint8_t *state, int n, int max_m, size_t row_bytes, D1Config cfg, D1Tables tab, const int64_t *actions,
    uint8_t *obs, float *out, uint32_t *hash, const uint8_t *active) {
    __shared__ Smem sm;
    __shared__ D1Config lcfg;
    for (int i = lane_id(); i < (int)(sizeof(D1Config) / 4); i += 64) ((uint32_t *)&lcfg)[i] = ((const uint32_t *)&cfg)[i];
    __syncthreads();
    step_worlds<RM, STEP_WPB, false>(sm, state, n, max_m, row_bytes, &lcfg, tab, actions, obs, out, hash, active);
}
template <int RM>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(6))) void k_step_crowd(
    uint8_t *state, int n, int max_m, size_t row_bytes, D1Config cfg, D1Tables tab, const int64_t *actions,
    uint8_t *obs, float *out, uint32_t *hash, const uint8_t *active) {
    __shared__ Smem sm;
    step_worlds<RM, CROWD_WPB, true>(sm, state, n, max_m, row_bytes, &cfg, tab, actions, obs, out, hash, active);
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
            uint32_t f = 0, r = 0, l0 = 0, l1 = 0;
            for (int b = 0; b < 32 && 32 * j + b < W; b++) {
                int p = y * W + 32 * j + b;
                const int d = map.dist[p];
                f |= (uint32_t)(map.floor[p] != 0) << b;
                r |= (uint32_t)(d != 65535) << b;
                l0 |= (uint32_t)(d != 65535 && d % 3 == 1) << b;
                l1 |= (uint32_t)(d != 65535 && d % 3 == 2) << b;
            }
            sm->floor[y * RW + j] = f;
            sm->reach[y * RW + j] = r;
            sm->lay0[y * RW + j] = l0;
            sm->lay1[y * RW + j] = l1;
            sm->occ[y * RW + j] = 0;
            sm->front[y * RW + j] = 0;
        }
    }
    __syncthreads();
}
// the static field's layer of cell p (FAR where it is unreached)
__device__ __forceinline__ int wait_layer(const D1WaitMap &map, int p) {
    const int d = p >= 0 && p < N ? map.dist[p] : 65535;
    return d == 65535 ? FAR : d;
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
    if (x.lane < count) { occ_set_lane(x, x.mpos); x.mlay = wait_layer(map, x.mpos); }
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
    while (x.hp > 0 && ballot(mine && x.menergy >= 80)) {   // no reduction once nobody can act
        const int key = wave_max(mine && x.menergy >= 80 ? x.menergy * 128 + 127 - x.lane : -1);
        act(x, 127 - (key & 127));
    }
}
__device__ __forceinline__ uint32_t wait_digest(Ctx &x, int count) {
    uint32_t h = x.lane < count ? term((uint16_t)x.mpos | (uint32_t)(uint16_t)x.menergy << 16, 100 + x.lane) : 0u;
    h = wave_sum(h);
    return h + term((uint32_t)x.hp, 0) + term((uint32_t)x.regen, 1) + term((uint32_t)x.blocks, 2) +
           term((uint32_t)x.episode, 3) + term((uint32_t)x.g.pcg_state(), 4) + term((uint32_t)(x.g.pcg_state() >> 32), 5);
}
__device__ __forceinline__ void wait_load(Ctx &x, const D1WaitMap &map, const uint8_t *row, int count, int &fixture) {
    WaitHdr h = *(const WaitHdr *)row;
    x.g.pcg_load(h.rng_state, h.rng_inc);
    x.hp = h.hp; x.regen = h.regen; x.blocks = h.blocks; x.episode = h.episode; fixture = h.fixture;
    x.mpos = -1; x.menergy = -30000; x.mkind = x.lane % 6; x.mhp = 1; x.mawake = 1;
    if (x.lane < count) {
        const int16_t *m = (const int16_t *)(row + 64) + 2 * x.lane;
        x.mpos = m[0]; x.menergy = m[1];
        occ_set_lane(x, x.mpos);
    }
    x.mlay = x.lane < count ? wait_layer(map, x.mpos) : FAR;
    __syncthreads();
}
__device__ __forceinline__ void wait_store(Ctx &x, uint8_t *row, int count, int fixture) {
    if (x.lane == 0) {
        WaitHdr h{};
        h.rng_state = x.g.pcg_state(); h.rng_inc = x.g.inc;
        h.hp = x.hp; h.regen = x.regen; h.blocks = x.blocks; h.fixture = fixture; h.episode = x.episode;
        *(WaitHdr *)row = h;
    }
    if (x.lane < count) {
        int16_t *m = (int16_t *)(row + 64) + 2 * x.lane;
        m[0] = (int16_t)x.mpos; m[1] = (int16_t)x.menergy;
    }
}
__device__ __forceinline__ void wait_ctx(Ctx &x, Smem *sm, const D1Config *cfg, const D1WaitMap &map) {
    x.sm = sm; x.c = cfg; x.rays = nullptr; x.nslots = 0; x.lane = lane_id();
    x.player = map.player;
    set_view(x, 0, 0, 0, 0);
    x.mlay = FAR;
    x.lastl = 65535;   // the static field holds every reachable cell
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
    wait_load(x, map, row, count, fixture);
    for (int k = 0; k < steps; k++) {
        wait_step(x, map, count, fixture);
        if (trace) {
            uint32_t h = wait_digest(x, count);
            if (x.lane == 0) trace[(size_t)w * steps + k] = h;
        }
    }
    wait_store(x, row, count, fixture);
}

// ---------------------------------------------------------------- LOS table compiler
// Workgroup (row y, map m) flattens the view of the 80 origins of row y: the player
// field-of-view scan at each origin, then lane w < 10 packs bitset word w
// (bit (dy+8)*17+dx+8; offsets beyond 7 are never visible with inside blockers).
__global__ __launch_bounds__(64) void k_los_table(const uint8_t *floor, const uint64_t *rays, int nslots,
                                                  uint32_t *los) {
    __shared__ Smem sm;
    const int y = blockIdx.x, m = blockIdx.y;
    Ctx x;
    x.sm = &sm; x.c = nullptr; x.rays = rays; x.nslots = nslots; x.lane = lane_id();
    const uint8_t *f = floor + (size_t)m * N;
    for (int s = 0; s < 2; s++) {
        int yy = x.lane + 64 * s;
        if (yy >= H) break;
        for (int j = 0; j < 3; j++) {
            uint32_t w = 0;
            for (int b = 0; b < 32 && 32 * j + b < W; b++) w |= (uint32_t)(f[yy * W + 32 * j + b] != 0) << b;
            sm.floor[yy * RW + j] = w;
        }
    }
    __syncthreads();
    for (int xx = 0; xx < W; xx++) {
        x.player = y * W + xx;
        compute_view(x);
        if (x.lane < 10) {
            uint32_t word = 0;
            for (int b = 0; b < 32; b++) {
                int idx = 32 * x.lane + b;
                if (idx < 289 && vis_rel(x, idx % 17 - 8, idx / 17 - 8)) word |= 1u << b;
            }
            los[((size_t)m * N + x.player) * 10 + x.lane] = word;
        }
    }
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

// ---------------------------------------------------------------- v1 pursuit controller
// The v1 task's scripted controller (gpu-d1/src/learn.cu:599-621, bound by
// gpu-d1/scripts/learn_env.py:114 as heuristic()): attack the weakest adjacent living monster
// (lowest HP, the first direction N, E, S, W, NE, SE, SW, NW among equals); otherwise take as
// target the nearest living monster by floor distance (the lowest index among the nearest)
// and step to the first neighbour, in direction order, that is one step closer to it; wait
// when no living monster is reachable. Distances are 8-connected BFS layers over the world's
// floor bitmap, as the reference's all-pairs distance rows are (learn_env.py:31-39). One
// world per wave, lane l holding map rows l and 64 + l: the search from the player stops at
// the first layer L that holds a living monster, the search from the target runs L - 1
// layers, and the player's neighbours in that last layer are the ones one step closer.
// The result is a v1 action (0-7 bump, 8 wait) or, with `joint`, this build's joint action
// for it on the same world (a bump into a living monster's cell is ATTACK d, 8 + d; any
// other direction MOVE d; 8 is WAIT, 16).
__device__ __forceinline__ bool bfs_layer(Row &f0, Row &f1, Row &r0, Row &r1, const Row &fl0, const Row &fl1,
                                          int lane) {
    const bool has1 = lane < H - 64;
    const Row zero{0, 0, 0};
    const Row f0_63 = row_lane(f0, 63), f1_0 = row_lane(f1, 0);
    const Row u0 = row_sel(lane == 0, zero, row_up(f0)), d0 = row_sel(lane == 63, f1_0, row_dn(f0));
    const Row u1 = row_sel(lane == 0, f0_63, row_up(f1)), d1 = row_sel(lane >= H - 65, zero, row_dn(f1));
    const Row n0 = row_andn(row_and(dilate(f0, u0, d0), fl0), r0);
    const Row n1 = has1 ? row_andn(row_and(dilate(f1, u1, d1), fl1), r1) : zero;
    r0 = row_or(r0, n0);
    r1 = row_or(r1, n1);
    f0 = n0;
    f1 = n1;
    return ballot(row_any(n0) || row_any(n1)) != 0;
}
// direction of the unit offset (dx, dy): nibble 3(dy + 1) + dx + 1 of the table
__device__ __forceinline__ int dir_of(int dx, int dy) {
    constexpr uint64_t T = 7ull | 0ull << 4 | 4ull << 8 | 3ull << 12 | 1ull << 20 | 6ull << 24 | 2ull << 28 | 5ull << 32;
    return (int)((T >> (4 * (3 * (dy + 1) + dx + 1))) & 15u);
}
__global__ __launch_bounds__(64) void k_heuristic_v1(const uint8_t *state, int n, int max_m, size_t row_bytes,
                                                     int count, int joint, int64_t *actions) {
    __shared__ uint32_t bm[ROWS_WORDS];   // the living monsters' cells, later one search layer
    const int env = blockIdx.x;           // grid = n
    const int lane = lane_id();
    const bool has1 = lane < H - 64;
    const Row zero{0, 0, 0};
    const uint8_t *row = state + (size_t)env * row_bytes;
    const int player = ((const Hdr *)row)->player;
    const int px = player % W, py = player / W;
    int mpos = -1, mhp = 0;
    if (lane < count) {
        const Mon m = ((const Mon *)(row + OFF_MON))[lane];
        mpos = m.pos;
        mhp = m.hp;
    }
    const bool alive = lane < count && mhp > 0;
    // the weakest adjacent living monster: HP x 8 + direction, least over the monster lanes
    int key = 1 << 30;
    if (alive) {
        const int dx = mpos % W - px, dy = mpos / W - py;
        if (iabs(dx) <= 1 && iabs(dy) <= 1) key = mhp * 8 + dir_of(dx, dy);
    }
    key = wave_min(key);
    int a = 8;
    if (key < (1 << 30)) {
        a = key & 7;
    } else {
        row_st(bm, lane, zero);
        if (has1) row_st(bm, 64 + lane, zero);
        __syncthreads();
        if (alive) atomicOr(&bm[(mpos / W) * RW + ((mpos % W) >> 5)], 1u << ((mpos % W) & 31));
        __syncthreads();
        const Row mv0 = row_ld(bm, lane), mv1 = has1 ? row_ld(bm, 64 + lane) : zero;
        const uint32_t *fg = (const uint32_t *)(row + off_floor(max_m));
        const Row fl0 = row_ld(fg, lane), fl1 = has1 ? row_ld(fg, 64 + lane) : zero;
        const Row pb = row_range(px, px);
        Row f0 = lane == py ? pb : zero, f1 = has1 && 64 + lane == py ? pb : zero;
        Row r0 = f0, r1 = f1;
        int L = 0;
        bool found = false;
        // every layer adds a cell, so the search ends within the map's cell count
        while (bfs_layer(f0, f1, r0, r1, fl0, fl1, lane)) {
            L++;
            if (ballot(row_any(row_and(f0, mv0)) || row_any(row_and(f1, mv1)))) {
                found = true;
                break;
            }
        }
        if (found) {
            __syncthreads();
            row_st(bm, lane, row_and(f0, mv0));
            if (has1) row_st(bm, 64 + lane, row_and(f1, mv1));
            __syncthreads();
            const uint64_t hits = ballot(alive && bit(bm, mpos));
            const int target = lane_val(mpos, __ffsll((unsigned long long)hits) - 1);
            const int tx = target % W, ty = target / W;
            const Row tb = row_range(tx, tx);
            f0 = lane == ty ? tb : zero;
            f1 = has1 && 64 + lane == ty ? tb : zero;
            r0 = f0;
            r1 = f1;
            for (int k = 0; k < L - 1; k++) bfs_layer(f0, f1, r0, r1, fl0, fl1, lane);
            __syncthreads();
            row_st(bm, lane, f0);
            if (has1) row_st(bm, 64 + lane, f1);
            __syncthreads();
            const int q = lane < 8 ? nbr(player, lane) : -1;
            const uint64_t closer = ballot(q >= 0 && bit(bm, q));
            if (closer) a = __ffsll((unsigned long long)closer) - 1;
        }
    }
    if (joint) {
        const int q = a < 8 ? nbr(player, a) : -1;
        const bool bump = ballot(alive && q >= 0 && mpos == q) != 0;
        a = a == 8 ? 16 : bump ? 8 + a : a;
    }
    if (lane == 0) actions[env] = a;
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

int d1_los_table(const uint8_t *floor, int n_maps, const D1Tables *rays, uint32_t *los, void *stream) {
    if (n_maps < 0 || !floor || !los || !rays || !rays->ray_slots || rays->nslots < 1 || rays->nslots > 64)
        return D1_E_ARG;
    if (n_maps == 0) return 0;
    hipLaunchKernelGGL(d1::k_los_table, dim3(d1::H, n_maps), dim3(64), 0, (hipStream_t)stream, floor,
                       rays->ray_slots, rays->nslots, los);
    return (int)hipGetLastError();
}
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
int d1_heuristic(const void *state, int n, int max_monsters, const D1Config *cfg, int joint, int64_t *actions,
                 void *stream) {
    if (n < 0 || max_monsters < 1 || max_monsters > D1_MAX_MONSTERS || !cfg || cfg->count < 0 ||
        cfg->count > max_monsters || (joint != 0 && joint != 1))
        return D1_E_ARG;
    if (!state || !actions) return D1_E_ARG;
    if (n == 0) return 0;
    hipLaunchKernelGGL(d1::k_heuristic_v1, dim3(n), dim3(64), 0, (hipStream_t)stream, (const uint8_t *)state, n,
                       max_monsters, (size_t)d1::state_bytes(max_monsters), cfg->count, joint, actions);
    return (int)hipGetLastError();
}
int d1_step(void *state, int n, int max_monsters, const D1Config *cfg, const D1Tables *tab, const int64_t *actions,
            uint8_t *obs, float *out, uint32_t *hash, const uint8_t *active, void *stream) {
    int e = d1::validate(n, max_monsters, cfg, tab);
    if (e) return e;
    if (!state || !actions) return D1_E_ARG;
    if (n == 0) return 0;
    auto kern = max_monsters > 8 ? (cfg->rng_mode == 0 ? d1::k_step_crowd<0> : d1::k_step_crowd<1>)
                                 : (cfg->rng_mode == 0 ? d1::k_step<0> : d1::k_step<1>);
    const int wpb = max_monsters > 8 ? d1::CROWD_WPB : d1::STEP_WPB;
    const int tail = max_monsters > 8 ? d1::CROWD_TAIL : d1::STEP_TAIL;
    hipLaunchKernelGGL(kern, dim3(d1::step_blocks(n, wpb, tail)), dim3(64), 0, (hipStream_t)stream,
                       (uint8_t *)state, n, max_monsters,
                       (size_t)d1::state_bytes(max_monsters), *cfg, *tab, actions, obs, out, hash, active);
    return (int)hipGetLastError();
}
}
