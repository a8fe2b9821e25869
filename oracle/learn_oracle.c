/* TEST INFRASTRUCTURE ONLY — CPU restatement of the reference's d1-stairs-v2
 * learning task, the checker for the HIP library's learn_* entry points.
 *
 * Scalar, one world at a time, with the reference's full-size per-cell arrays and
 * its FIFO breadth-first searches, written from
 *   gpu-d1/branches/d1-stairs-v2/src/learn.cu   (task: reset, reveal, frontier list,
 *                                                encounter slots, observation, mask,
 *                                                joint actions, heuristic controller)
 *   gpu-d1/src/sim.h                            (melee, scheduler, monster pathing)
 * for the build of gpu-d1/branches/d1-stairs-v2/scripts/assets.py:5 (24 enemies, no
 * ogres, KILL/DEATH/EXPLORE 0, CLEAR 1000 milli, TURN_COST 1e-5, PROGRESS_INPUT 2,
 * LOS waking, MULTI_MAP). The monster distance field is read from the tables'
 * all-pairs rows as the reference does; the HIP library recomputes it by BFS, so
 * agreement also checks that substitution. Compile with -ffp-contract=off.
 * Only tests/ load this; the product never links it.
 *
 * Parity unpinned (no reference log or fixture fixes them): the values that lo_reset's
 * clump anchors and stairs reservoir draw from their RNG copies (the player and monster
 * draws before them are the v1 order that the reference's recorded v1 run pins; what
 * sampling fixes about the clumps and stairs is pinned in tests/test_reset_pins.py: no
 * draw from the play stream, bounds reached, uniform choices). lo_heuristic_one's priority
 * order is pinned by worlds in which two of its rules apply at once
 * (tests/test_learn_oracle.py::test_controller_priority_order).
 */
#include "d1_oracle.h"
#include "../include/d1learn.h"
#include <stddef.h>
#include <string.h>

#define W O_W
#define H O_H
#define N O_N
#define LE O_LE
#define REQ D1L_REQUIRED
#define VR 7
#define SIDE 15
#define VC 225
#define RR 8
#define PLAYER_OBS (2 * VC + LE * 5)   /* 650 */
#define BASE_OBS (PLAYER_OBS + 4)      /* 654 */
#define FRONTIER_OBS (BASE_OBS + 8 * RR)
#define VISIBLE_OBS (FRONTIER_OBS + 15)
#define ORIGINAL_OBS (VISIBLE_OBS + VC) /* 958 */
#define SLEEP_OBS (ORIGINAL_OBS + 1)
#define STAIR_OBS (SLEEP_OBS + LE)      /* 999 */
#define CLEAR_MILLI 1000
#define TURN_COST 0.00001f

static inline int imin(int a, int b) { return a < b ? a : b; }
static inline int imax(int a, int b) { return a > b ? a : b; }
static inline int iabs(int a) { return a < 0 ? -a : a; }
static inline int cheb(int a, int b) { return imax(iabs(a % W - b % W), iabs(a / W - b / W)); }
static const int DX[8] = {0, 1, 0, -1, 1, 1, -1, -1};
static const int DY[8] = {-1, 0, 1, 0, -1, 1, 1, -1};
static inline int nb(int p, int d) {
    int x = p % W + DX[d], y = p / W + DY[d];
    return x >= 0 && x < W && y >= 0 && y < H ? y * W + x : -1;
}

/* ------------------------------------------------------------------ tables (learn.cu:155-190) */
static inline int floor_at(const D1LTables *t, int m, int p) { return p >= 0 && p < N && t->floor[(size_t)m * N + p]; }
static inline const int16_t *cells_of(const D1LTables *t, int m) { return t->cells + (size_t)m * N; }
static inline const uint16_t *field_of(const D1LTables *t, int m, int player) {
    int row = t->index[(size_t)m * N + player];
    return t->distance + ((size_t)t->distance_offsets[m] + (size_t)row) * N;
}
static inline int los_bit(const D1LTables *t, int m, int origin, int dx, int dy) {
    int bit = (dy + 8) * 17 + dx + 8;
    return (t->los[((size_t)m * N + origin) * 10 + bit / 32] >> (bit % 32)) & 1;
}

/* learn.cu:192-198: the player's 15x15 LOS */
int lo_in_view(const LState *s, const D1LTables *t, int p) {
    if (p < 0 || p >= N) return 0;
    int dx = p % W - s->player % W, dy = p / W - s->player / W;
    if (iabs(dx) > VR || iabs(dy) > VR) return 0;
    return los_bit(t, s->map_id, s->player, dx, dy);
}
#define in_view lo_in_view
/* learn.cu:201-207: a monster's LOS to the player within Chebyshev 6 (waking only) */
static int detects(const LState *s, const D1LTables *t, int origin) {
    int dx = s->player % W - origin % W, dy = s->player / W - origin / W;
    if (iabs(dx) > 6 || iabs(dy) > 6) return 0;
    return los_bit(t, s->map_id, origin, dx, dy);
}
static int visible_enemy(const LState *s, const D1LConfig *c, const D1LTables *t) {   /* :208-211 */
    for (int i = 0; i < c->count; i++)
        if (s->mhp[i] > 0 && in_view(s, t, s->pos[i])) return 1;
    return 0;
}
static int visible_awake(const LState *s, const D1LConfig *c, const D1LTables *t) {   /* :448-451 */
    for (int i = 0; i < c->count; i++)
        if (s->mhp[i] > 0 && s->awake[i] && in_view(s, t, s->pos[i])) return 1;
    return 0;
}
/* learn.cu:212-218: sightings mark an enemy encountered and give it the next slot */
static void update_knowledge(LState *s, const D1LConfig *c, const D1LTables *t) {
    for (int i = 0; i < c->count; i++) {
        if (s->mhp[i] <= 0) continue;
        int vis = in_view(s, t, s->pos[i]);
        if (vis) s->encountered[i] = 1;
        if (vis && s->enemy_slot[i] < 0) s->enemy_slot[i] = (int16_t)s->next_slot++;
    }
}

/* ------------------------------------------------------------------ known-floor BFS (learn.cu:222-266) */
/* FIFO BFS from the player over viewed floor. nearest_only stops when the first
 * frontier anchor is dequeued (the whole nearest layer is discovered by then) and
 * returns at once without anchors. */
void lo_known_distances(const LState *s, const D1LTables *t, uint16_t *ds, int nearest_only) {
    static __thread int16_t queue[N];
    for (int p = 0; p < N; p++) ds[p] = 65535;
    int head = 0, tail = 1;
    queue[0] = (int16_t)s->player;
    ds[s->player] = 0;
    if (nearest_only && s->frontier_count == 0) return;
    while (head < tail) {
        int p = queue[head++];
        int slot = s->frontier_slot[p];
        if (nearest_only && slot >= 0 && slot < s->frontier_count && s->frontier_cells[slot] == p) break;
        for (int d = 0; d < 8; d++) {
            int q = nb(p, d);
            if (q >= 0 && s->viewed[q] && floor_at(t, s->map_id, q) && ds[q] == 65535) {
                ds[q] = (uint16_t)(ds[p] + 1);
                queue[tail++] = (int16_t)q;
            }
        }
    }
}
/* Walk the distance field back from the target; the first-found predecessor in
 * direction order is taken; returns the player's direction toward it, or -1. */
int lo_route_first_step(int player, int target, const uint16_t *ds) {
    if (target < 0 || ds[target] == 65535 || target == player) return -1;
    int p = target;
    while (ds[p] > 1) {
        int prev = -1;
        for (int d = 0; d < 8; d++) {
            int q = nb(p, d);
            if (q >= 0 && (int)ds[q] + 1 == (int)ds[p]) { prev = q; break; }
        }
        if (prev < 0) return -1;
        p = prev;
    }
    for (int d = 0; d < 8; d++) if (nb(player, d) == p) return d;
    return -1;
}

/* ------------------------------------------------------------------ frontier list + reveal (learn.cu:269-336) */
/* An anchor is seen floor with an in-bounds neighbour never viewed (wall or floor). */
static int frontier_anchor(const LState *s, const D1LTables *t, int p) {
    if (p < 0 || !floor_at(t, s->map_id, p) || !s->seen[p]) return 0;
    for (int d = 0; d < 8; d++) {
        int q = nb(p, d);
        if (q >= 0 && !s->viewed[q]) return 1;
    }
    return 0;
}
/* Insert by appending; delete by moving the last entry into the hole. */
void lo_refresh_frontier(LState *s, const D1LTables *t, int p) {
    if (p < 0) return;
    int want = frontier_anchor(s, t, p), slot = s->frontier_slot[p];
    if (want && slot < 0) {
        int n = s->frontier_count++;
        s->frontier_cells[n] = (int16_t)p;
        s->frontier_slot[p] = (int16_t)n;
    } else if (!want && slot >= 0) {
        int last = --s->frontier_count;
        int q = s->frontier_cells[last];
        s->frontier_cells[slot] = (int16_t)q;
        s->frontier_slot[q] = (int16_t)slot;
        s->frontier_slot[p] = -1;
    }
}
/* Mark the view (row-major), then refresh each newly viewed cell followed by its
 * eight neighbours in direction order; returns the newly seen floor count. */
int lo_reveal(LState *s, const D1LTables *t) {
    int fresh = 0, nchanged = 0, changed[VC];
    for (int y = -VR; y <= VR; y++)
        for (int x = -VR; x <= VR; x++) {
            int px = s->player % W + x, py = s->player / W + y;
            if (px < 0 || px >= W || py < 0 || py >= H) continue;
            int p = py * W + px;
            if (!in_view(s, t, p)) continue;
            if (!s->viewed[p]) { s->viewed[p] = 1; changed[nchanged++] = p; }
            if (floor_at(t, s->map_id, p) && !s->seen[p]) { s->seen[p] = 1; fresh++; }
        }
    for (int i = 0; i < nchanged; i++) {
        lo_refresh_frontier(s, t, changed[i]);
        for (int d = 0; d < 8; d++) lo_refresh_frontier(s, t, nb(changed[i], d));
    }
    s->floor_seen += fresh;
    return fresh;
}
static int stair_index(const LState *s) {   /* learn.cu:338-341 */
    for (int k = 0; k < 3; k++) if (s->player == s->stairs[k]) return k + 1;
    return 0;
}
static int known_stairs(const LState *s) {   /* :342-344 */
    int n = 0;
    for (int k = 0; k < 3; k++) n += s->stairs[k] >= 0 && s->seen[s->stairs[k]] != 0;
    return n;
}
/* :345-350: the first remembered stair with the smallest known distance */
int lo_nearest_stair(const LState *s, const uint16_t *ds) {
    int best = -1, dist = 65535;
    for (int k = 0; k < 3; k++) {
        int p = s->stairs[k];
        if (p >= 0 && s->seen[p] && ds[p] < dist) { best = p; dist = ds[p]; }
    }
    return best;
}

/* Planted mistakes for the tests that show the reset pins bite (0 = none, the faithful
 * rules): 1 clumps and stairs drawn from the play stream instead of copies, 2 the stairs'
 * draw bound counting every cell of the list, not the eligible ones, 3 a clump member's
 * draw bound counting every direction, not the free neighbours, 4 anchors needing more
 * than two (not at least two) free neighbours. */
static int lplanted;
void lo_plant(int which) { lplanted = which; }

/* ------------------------------------------------------------------ reset (learn.cu:351-446) */
void lo_reset(LState *s, const D1LConfig *c, const D1LTables *t, int clump) {
    static const int MHP[6] = {8, 10, 12, 16, 12, 10};
    ORng *g = &s->rng;
    s->map_id = t->map_filter >= 0 ? t->map_filter : o_rng_r(g, t->n_maps);
    const int m = s->map_id, ncells = t->map_ncells[m];
    const int16_t *cells = cells_of(t, m);
    for (int p = 0; p < N; p++) s->occ[p] = -1;
    s->player = cells[o_rng_r(g, ncells)];
    s->hp = c->hp; s->regen = 0; s->blocks = 0;
    s->ticks = 0; s->decisions = 0; s->killed = 0; s->next_slot = 0; s->floor_seen = 0;
    for (int i = 0; i < LE; i++) { s->enemy_slot[i] = -1; s->encountered[i] = 0; }
    for (int i = 0; i < REQ; i++) {
        int p;
        do p = cells[o_rng_r(g, ncells)]; while (p == s->player || s->occ[p] >= 0);
        s->pos[i] = (int16_t)p; s->occ[p] = (int16_t)i; s->mhp[i] = (int16_t)MHP[i % 6];
        s->energy[i] = (int16_t)(70 + o_rng_r(g, 10));
        s->awake[i] = 0;
    }
    /* clumps of three from a copy of the RNG: a reservoir-chosen anchor with at least
     * two free floor neighbours, then two reservoir-chosen free neighbours */
    ORng place_copy = *g, *place = lplanted == 1 ? g : &place_copy;
    s->placement_clumped = clump == 2 || (clump == 1 && o_rng_r(place, 3) == 0);
    if (s->placement_clumped) {
        for (int i = 0; i < REQ; i++) s->occ[s->pos[i]] = -1;
        for (int i = 0; i < REQ; i += 3) {
            int anchor = -1, eligible = 0;
            for (int j = 0; j < ncells; j++) {
                int p = cells[j];
                if (p == s->player || s->occ[p] >= 0) continue;
                int free_nb = 0;
                for (int a = 0; a < 8; a++) {
                    int q = nb(p, a);
                    free_nb += floor_at(t, m, q) && q != s->player && s->occ[q] < 0;
                }
                if (free_nb >= (lplanted == 4 ? 3 : 2) && o_rng_r(place, ++eligible) == 0) anchor = p;
            }
            if (anchor < 0) { s->error = 1; return; }
            s->pos[i] = (int16_t)anchor; s->occ[anchor] = (int16_t)i;
            for (int k = 1; k <= 2; k++) {
                int chosen = -1, n = 0;
                for (int a = 0; a < 8; a++) {
                    int q = nb(anchor, a);
                    if (floor_at(t, m, q) && q != s->player && s->occ[q] < 0 &&
                        o_rng_r(place, lplanted == 3 ? a + 1 : ++n) == 0)
                        chosen = q;
                }
                if (chosen < 0) { s->error = 1; return; }
                s->pos[i + k] = (int16_t)chosen; s->occ[chosen] = (int16_t)(i + k);
            }
        }
    }
    memset(s->seen, 0, N);
    memset(s->viewed, 0, N);
    s->frontier_count = 0;
    for (int p = 0; p < N; p++) s->frontier_slot[p] = -1;
    /* three stairs from another copy: >= 12 from the player, >= 8 from earlier stairs */
    ORng st_copy = *g, *st = lplanted == 1 ? g : &st_copy;
    s->first_stair_tick = -1;
    for (int k = 0; k < 3; k++) {
        int selected = -1, count = 0;
        for (int j = 0; j < ncells; j++) {
            int p = cells[j];
            int ok = cheb(p, s->player) >= 12 && s->occ[p] < 0;
            for (int q = 0; q < k; q++) ok &= cheb(p, s->stairs[q]) >= 8;
            if (ok && o_rng_r(st, lplanted == 2 ? j + 1 : ++count) == 0) selected = p;
        }
        if (selected < 0) s->error = 1;
        s->stairs[k] = selected;
    }
    lo_reveal(s, t);   /* no reward for the initial view */
    update_knowledge(s, c, t);
}

/* ------------------------------------------------------------------ monsters (gpu-d1/src/sim.h:130-269) */
/* The learning-task world's view for the oracle's shared monster rules (o_m_*). */
static OMonsters learn_monsters(LState *s, const D1LConfig *c, const D1LTables *t) {
    OMonsters m = {&s->rng, &s->hp, &s->blocks, s->pos, s->energy, s->occ, t->floor + (size_t)s->map_id * N, NULL,
                   (const int32_t *)c->kinds, s->player, c->ac100, c->ev100, c->sh100, c->shield_limit, c->repair,
                   c->gdr[0], c->gdr[1]};
    return m;
}

/* ------------------------------------------------------------------ observation (learn.cu:480-682) */
static int ring_index(int x, int y) {
    if (y == -RR) return x + RR;
    if (y == RR) return 2 * RR + 1 + x + RR;
    if (x == -RR) return 2 * (2 * RR + 1) + y + RR - 1;
    return 2 * (2 * RR + 1) + (2 * RR - 1) + y + RR - 1;
}
void lo_observe(LState *s, const D1LConfig *c, const D1LTables *t, float *o, float *mask) {
    static __thread uint16_t ds[N];
    const int m = s->map_id, px = s->player % W, py = s->player / W;
    memset(o, 0, sizeof(float) * D1L_OBS);
    for (int y = -VR; y <= VR; y++)
        for (int x = -VR; x <= VR; x++) {
            int qx = px + x, qy = py + y, j = (y + VR) * SIDE + x + VR;
            if (qx < 0 || qx >= W || qy < 0 || qy >= H) continue;
            int p = qy * W + qx;
            o[j] = s->viewed[p] ? (floor_at(t, m, p) ? 1.f : -1.f) : 0.f;
            o[VISIBLE_OBS + j] = (float)in_view(s, t, p);
            int id = s->occ[p];
            if (id >= 0 && in_view(s, t, p)) o[VC + j] = s->mhp[id] / 16.f;
        }
    for (int i = 0; i < c->count; i++) {
        if (s->mhp[i] <= 0 || !in_view(s, t, s->pos[i])) continue;
        int j = 2 * VC + s->enemy_slot[i] * 5;
        o[j] = (s->pos[i] % W - px) / 80.f;
        o[j + 1] = (s->pos[i] / W - py) / 70.f;
        o[SLEEP_OBS + s->enemy_slot[i]] = s->awake[i] ? -1.f : 1.f;
        o[j + 2] = s->mhp[i] / 16.f;
        o[j + 3] = i >= REQ ? 1.2f : (i % 6) / 5.f;
        o[j + 4] = 1.f;
    }
    o[ORIGINAL_OBS] = s->floor_seen / 1024.f;
    o[PLAYER_OBS] = s->hp / (float)c->hp;
    o[PLAYER_OBS + 1] = s->ticks / 2048.f;
    o[PLAYER_OBS + 2] = px / 80.f;
    o[PLAYER_OBS + 3] = py / 70.f;
    for (int y = -RR; y <= RR; y++)
        for (int x = -RR; x <= RR; x++) {
            if (iabs(x) != RR && iabs(y) != RR) continue;
            int qx = px + x, qy = py + y;
            if (qx < 0 || qx >= W || qy < 0 || qy >= H) continue;
            int p = qy * W + qx;
            if (s->viewed[p]) o[BASE_OBS + ring_index(x, y)] = floor_at(t, m, p) ? 1.f : -1.f;
        }
    int ks = known_stairs(s);
    lo_known_distances(s, t, ds, ks == 0);
    int best = -1, best_dist = 65535, best_unseen = 0, best_dx = 0, best_dy = 0;
    for (int k = 0; k < s->frontier_count; k++) {
        int p = s->frontier_cells[k], d = ds[p];
        if (d >= best_dist) continue;
        best = p; best_dist = d; best_unseen = 0; best_dx = 0; best_dy = 0;
        for (int nd = 0; nd < 8; nd++) {
            int q = nb(p, nd);
            if (q >= 0 && !s->viewed[q] && ++best_unseen == 1) { best_dx = q % W - p % W; best_dy = q / W - p / W; }
        }
    }
    if (best >= 0) {
        float *f = o + FRONTIER_OBS;
        f[0] = 1.f;
        f[1] = (best % W - px) / (float)W;
        f[2] = (best / W - py) / (float)H;
        f[3] = best_dist / (float)(W + H);
        f[4] = best_unseen / 8.f;
        f[5] = (float)best_dx;
        f[6] = (float)best_dy;
        int dir = lo_route_first_step(s->player, best, ds);
        if (dir >= 0) f[7 + dir] = 1.f;
    }
    for (int d = 0; d < 8; d++) {
        int p = nb(s->player, d);
        int enemy = p >= 0 && in_view(s, t, p) && s->occ[p] >= 0;
        mask[d] = (float)(p >= 0 && (!s->viewed[p] || floor_at(t, m, p)) && !enemy);
        mask[8 + d] = (float)enemy;
    }
    mask[18] = (float)(stair_index(s) > 0);
    float *sb = o + STAIR_OBS;
    sb[0] = ks / 3.f;
    sb[15] = mask[18];
    if (ks) {
        int target = lo_nearest_stair(s, ds);
        if (target >= 0) {
            sb[1] = 1.f;
            sb[2] = (target % W - px) / (float)W;
            sb[3] = (target / W - py) / (float)H;
            sb[4] = ds[target] / (float)(W + H);
            int d = lo_route_first_step(s->player, target, ds);
            if (d >= 0) {
                int q = nb(s->player, d);
                sb[5] = (float)(q % W - px);
                sb[6] = (float)(q / W - py);
                sb[7 + d] = 1.f;
            }
        }
    }
    mask[16] = 1.f;
    mask[17] = (float)(s->hp < c->hp && c->regen > 0 && !visible_awake(s, c, t));
}

/* ------------------------------------------------------------------ one physical turn (learn.cu:684-828) */
static void primitive(LState *s, const D1LConfig *c, const D1LTables *t, int action, int limit, float *out, int clump) {
    memset(out, 0, sizeof(float) * D1L_OUT);
    int milli = 0;
    s->blocks = 0;
    s->regen += c->regen;
    while (s->regen >= 100) { s->hp = imin(c->hp, s->hp + 1); s->regen -= 100; }
    if (action >= 0 && action < 8) {
        int p = nb(s->player, action);
        if (floor_at(t, s->map_id, p)) {
            int id = s->occ[p];
            if (id >= 0) {
                s->encountered[id] = 1;
                if (s->enemy_slot[id] < 0) s->enemy_slot[id] = (int16_t)s->next_slot++;
                if (o_rng_r(&s->rng, 5) != 0) {
                    s->mhp[id] = (int16_t)(s->mhp[id] - (1 + o_rng_r(&s->rng, 4)));
                    if (s->mhp[id] <= 0) {
                        s->mhp[id] = 0; s->occ[p] = -1; s->energy[id] = -30000;
                        s->killed++;
                    }
                }
            } else s->player = p;
        }
    }
    lo_reveal(s, t);   /* EXPLORE_MILLI = 0: the reveal still updates memory and the frontier */
    out[41] = (float)visible_awake(s, c, t);
    out[33] = (float)visible_enemy(s, c, t);
    int clear = action == 18 && stair_index(s) > 0 && s->hp > 0;
    if (!clear) {
        for (int i = 0; i < c->count; i++)
            if (s->mhp[i] > 0 && !s->awake[i] && detects(s, t, s->pos[i])) { s->awake[i] = 1; s->energy[i] = 70; }
        for (int i = 0; i < c->count; i++)
            if (s->mhp[i] > 0 && !s->awake[i]) s->energy[i] = -30000;
        for (int i = 0; i < c->count; i++)
            if (s->mhp[i] > 0) s->energy[i] = (int16_t)(s->energy[i] + c->kinds[i % 6].speed);
        const uint16_t *dist = field_of(t, s->map_id, s->player);
        OMonsters mon = learn_monsters(s, c, t);
        while (s->hp > 0) {
            int id = o_m_scan(s->energy, c->count);
            if (id < 0) break;
            o_m_act(&mon, dist, id);
            if (in_view(s, t, s->pos[id])) { out[33] = 1.f; if (s->awake[id]) out[41] = 1.f; }
        }
    }
    s->ticks++;
    if (s->first_stair_tick < 0 && known_stairs(s) > 0) s->first_stair_tick = s->ticks;
    int death = s->hp <= 0, timeout = !clear && !death && s->ticks >= limit;
    if (clear) milli += CLEAR_MILLI;
    float reward = 0.001f * (float)milli;
    reward -= TURN_COST;
    out[26] = 1.f;
    out[33] = (float)(out[33] != 0.f || visible_enemy(s, c, t));
    out[41] = (float)(out[41] != 0.f || visible_awake(s, c, t));
    update_knowledge(s, c, t);
    for (int i = 0; i < REQ; i++) {
        out[8] += s->encountered[i] != 0;
        out[9] += s->mhp[i] > 0 && !s->encountered[i];
        out[10] += s->mhp[i] > 0 && s->encountered[i];
        out[12] += s->mhp[i] > 0 && in_view(s, t, s->pos[i]);
    }
    out[13] = (float)s->floor_seen;
    out[11] = out[13] / (float)t->map_ncells[s->map_id];
    out[42] = (float)known_stairs(s);
    out[43] = (float)s->first_stair_tick;
    out[44] = clear ? (float)stair_index(s) : 0.f;
    out[0] = reward; out[1] = (float)(clear || death || timeout); out[2] = (float)clear;
    out[3] = (float)s->killed; out[4] = (float)imax(0, s->hp); out[5] = (float)s->ticks;
    out[6] = (float)death; out[7] = (float)timeout;
    if (out[1] != 0.f) { s->episode++; lo_reset(s, c, t, clump); }
}
/* learn.cu:853-875: MOVE 0-7, ATTACK 8-15, WAIT 16, REST 17 (waits until healed or
 * an awake enemy is seen), DESCEND 18; an invalid action is one wait. */
void lo_transition(LState *s, const D1LConfig *c, const D1LTables *t, int action, int limit, float *out, int clump) {
    int decisions = s->decisions + 1, initial_hp = s->hp, elapsed = 0, interrupted = 0, invalid = 0;
    float total = 0.f, discounted = 0.f, factor = 1.f, exposure[3] = {0.f, 0.f, 0.f};
    for (;;) {
        int d = 8;
        if (action >= 0 && action < 16) {
            int dir = action % 8, p = nb(s->player, dir);
            int enemy = p >= 0 && in_view(s, t, p) && s->occ[p] >= 0;
            int valid = action < 8 ? p >= 0 && (!s->viewed[p] || floor_at(t, s->map_id, p)) && !enemy : enemy;
            if (valid) d = dir; else invalid = 1;
        } else if (action == 17) invalid = s->hp >= c->hp || visible_awake(s, c, t) || c->regen <= 0;
        else if (action == 18) { if (stair_index(s) > 0) d = 18; else invalid = 1; }
        else if (action != 16) invalid = 1;
        primitive(s, c, t, d, limit, out, clump);
        elapsed++;
        total += out[0];
        discounted += factor * out[0];
        factor *= 1.f;
        for (int k = 0; k < 3; k++) exposure[k] += out[21 + k];
        if (out[1] != 0.f || invalid || action != 17) break;
        interrupted = out[41] != 0.f;
        if (interrupted || s->hp >= c->hp) break;
    }
    out[0] = total; out[40] = discounted; out[26] = (float)elapsed;
    for (int k = 0; k < 3; k++) out[21 + k] = exposure[k];
    if (action == 17) {
        out[34] = 1.f; out[35] = (float)elapsed; out[36] = (float)(out[1] == 0.f && s->hp >= c->hp);
        out[37] = (float)interrupted; out[38] = (float)invalid; out[39] = (float)imax(0, (int)out[4] - initial_hp);
    }
    if (out[1] == 0.f) s->decisions = decisions;
}

/* ------------------------------------------------------------------ controller (learn.cu:452-479,876-888) */
static int adjacent_attack(const LState *s, const D1LTables *t) {
    int best = -1, hp = 100000;
    for (int d = 0; d < 8; d++) {
        int p = nb(s->player, d);
        if (p < 0) continue;
        int id = s->occ[p];
        if (id >= 0 && s->mhp[id] > 0 && in_view(s, t, p) && s->mhp[id] < hp) { hp = s->mhp[id]; best = d; }
    }
    return best;
}
static int engage_step(const LState *s, const D1LConfig *c, const D1LTables *t) {
    static __thread uint16_t ds[N];
    if (!visible_enemy(s, c, t)) return -1;
    lo_known_distances(s, t, ds, 0);
    int target = -1, bd = 65535;
    for (int slot = 0; slot < LE; slot++)
        for (int i = 0; i < c->count; i++)
            if (s->enemy_slot[i] == slot && s->mhp[i] > 0 && in_view(s, t, s->pos[i]) && ds[s->pos[i]] < bd) {
                target = s->pos[i]; bd = ds[target];
            }
    int d = lo_route_first_step(s->player, target, ds);
    if (d < 0) return -1;
    int q = nb(s->player, d);
    if (q < 0 || (s->occ[q] >= 0 && in_view(s, t, q))) return -1;
    return d;
}
static int explore_step(const LState *s, const D1LConfig *c, const D1LTables *t) {
    static __thread uint16_t ds[N];
    if (visible_enemy(s, c, t)) return -1;
    lo_known_distances(s, t, ds, 1);
    int best = -1, bd = 65535;
    for (int k = 0; k < s->frontier_count; k++) {
        int p = s->frontier_cells[k];
        if (ds[p] < bd) { best = p; bd = ds[p]; }
    }
    if (best < 0) return -1;
    if (best != s->player) return lo_route_first_step(s->player, best, ds);
    for (int d = 0; d < 8; d++) {
        int q = nb(s->player, d);
        if (q >= 0 && !s->viewed[q]) return d;
    }
    return -1;
}
/* learn.cu:881-886: the first step of the known-floor route to the nearest remembered stair,
 * unless a visible monster holds that cell; -1 when there is none */
static int stair_route(LState *s, const D1LTables *t, uint16_t *ds) {
    if (!known_stairs(s)) return -1;
    lo_known_distances(s, t, ds, 0);
    int d = lo_route_first_step(s->player, lo_nearest_stair(s, ds), ds);
    if (d < 0) return -1;
    int p = nb(s->player, d);
    return s->occ[p] >= 0 && in_view(s, t, p) ? -1 : d;
}
/* learn.cu:876-888, in its order: descend, attack, rest, wait, stair route, engage,
 * explore, wait. Planted priority swaps for the tests (lplanted): 10 the attack before the
 * descent, 11 the rest before the attack, 12 the wait before the attack, 13 the stair route
 * before the rest, 14 the stair route before the wait, 15 the engage step before the stair
 * route. */
int lo_heuristic_one(LState *s, const D1LConfig *c, const D1LTables *t) {
    static __thread uint16_t ds[N];
    const int pl = lplanted;
    int d;
    if (pl == 10 && (d = adjacent_attack(s, t)) >= 0) return 8 + d;
    if (stair_index(s) > 0) return 18;
    const int rest = s->hp < c->hp && c->regen > 0 && !visible_awake(s, c, t);
    if (pl == 11 && rest) return 17;
    if (pl == 12 && visible_awake(s, c, t)) return 16;
    d = adjacent_attack(s, t);
    if (d >= 0) return 8 + d;
    if (pl == 13 && (d = stair_route(s, t, ds)) >= 0) return d;
    if (rest) return 17;
    if (pl == 14 && (d = stair_route(s, t, ds)) >= 0) return d;
    if (visible_awake(s, c, t)) return 16;
    if (pl == 15 && (d = engage_step(s, c, t)) >= 0) return d;
    d = stair_route(s, t, ds);
    if (d >= 0) return d;
    d = engage_step(s, c, t);
    if (d >= 0) return d;
    d = explore_step(s, c, t);
    return d >= 0 ? d : 16;
}

/* ------------------------------------------------------------------ batch API */
int lo_state_bytes(void) { return (int)sizeof(LState); }
int lo_field_offset(int k) {
    static const size_t off[] = {
        offsetof(LState, rng), offsetof(LState, map_id), offsetof(LState, stairs), offsetof(LState, pos),
        offsetof(LState, energy), offsetof(LState, mhp), offsetof(LState, awake), offsetof(LState, enemy_slot),
        offsetof(LState, encountered), offsetof(LState, occ), offsetof(LState, seen), offsetof(LState, viewed),
        offsetof(LState, frontier_cells), offsetof(LState, frontier_slot), sizeof(LState)};
    return k >= 0 && k < (int)(sizeof off / sizeof off[0]) ? (int)off[k] : -1;
}
int lo_init(LState *st, int n, const D1LConfig *c, const D1LTables *t, uint64_t seed, float *obs, float *mask,
            int clump, int threads) {
    int err = 0;
    if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static) reduction(| : err)
    for (int i = 0; i < n; i++) {
        LState *s = &st[i];
        memset(s, 0, sizeof *s);
        o_pcg_seed(&s->rng, o_mix(seed + (uint64_t)i), (uint64_t)i + 1);
        D1LTables first = *t;
        if (first.map_filter == -2) first.map_filter = i % first.n_maps;
        lo_reset(s, c, &first, clump);
        lo_observe(s, c, t, obs + (size_t)i * D1L_OBS, mask + (size_t)i * D1L_ACTIONS);
        err |= s->error;
    }
    return err ? -2 : 0;
}
int lo_step(LState *st, int n, const D1LConfig *c, const D1LTables *t, const int64_t *actions, int limit,
            float *obs, float *mask, float *out, const uint8_t *active, int clump, int threads) {
    int err = 0;
    if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static) reduction(| : err)
    for (int i = 0; i < n; i++) {
        if (active && !active[i]) continue;
        lo_transition(&st[i], c, t, (int)actions[i], limit, out + (size_t)i * D1L_OUT, clump);
        lo_observe(&st[i], c, t, obs + (size_t)i * D1L_OBS, mask + (size_t)i * D1L_ACTIONS);
        err |= st[i].error;
    }
    return err ? -2 : 0;
}
int lo_heuristic(LState *st, int n, const D1LConfig *c, const D1LTables *t, int64_t *actions, int threads) {
    if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int i = 0; i < n; i++) actions[i] = lo_heuristic_one(&st[i], c, t);
    return 0;
}
/* All-pairs floor BFS rows for the cells list, as the reference's table builders do
 * (gpu-d1/scripts/learn_env.py:24-36, gpu-d1/scripts/compile_corpus.py:29-53). */
void lo_distance_table(const uint8_t *floor, const int16_t *cells, int ncells, uint16_t *out) {
#pragma omp parallel for schedule(dynamic, 16)
    for (int i = 0; i < ncells; i++) {
        int16_t queue[N];
        uint16_t *ds = out + (size_t)i * N;
        for (int p = 0; p < N; p++) ds[p] = 65535;
        int head = 0, tail = 1;
        queue[0] = cells[i];
        ds[cells[i]] = 0;
        while (head < tail) {
            int p = queue[head++];
            for (int d = 0; d < 8; d++) {
                int q = nb(p, d);
                if (q >= 0 && floor[q] && ds[q] == 65535) { ds[q] = (uint16_t)(ds[p] + 1); queue[tail++] = (int16_t)q; }
            }
        }
    }
}
/* The 5600 x 10 LOS bitsets of one byte map (o_los_bitset per origin). */
void lo_los_table(const uint8_t *floor, uint32_t *out) {
#pragma omp parallel for schedule(static)
    for (int p = 0; p < N; p++) o_los_bitset(floor, p, out + (size_t)p * 10);
}
