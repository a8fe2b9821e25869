/* TEST INFRASTRUCTURE ONLY — CPU restatement of the reference D:1 rules.
 *
 * Scalar, array-of-structs, one world at a time, written from the rules of
 *   gpu-d1/src/sim.h                                   (RNG, melee, scheduler, pathing)
 *   gpu-d1/branches/d1-stairs-v2/src/learn.cu          (joint actions, LOS view and
 *                                                       waking, stairs, reset, reveal)
 *   gpu-d1/src/learn.cu                                (v1 clear-on-kill-all, rewards)
 *   gpu-d1/scripts/compile_fixture.py:31-48            (ray LOS flattening)
 * plus the build's own specs for what the reference does not have: the room and
 * corridor level generator, the Philox counter RNG mode, the uint8 15x15x8
 * observation and the state hash. It is the checker for the HIP library; the
 * product never links it. Compile with -ffp-contract=off (reward arithmetic is
 * compared bit for bit).
 *
 * Parity unpinned: the values that reset's stairs reservoir draws (from an RNG copy after
 * the monster draws): no reference log records a stairs reset. What sampling fixes about
 * it is pinned (tests/test_reset_pins.py): it draws nothing from the play stream, its
 * eligibility bounds are reached and never crossed, and its choice is uniform over the
 * eligible cells. The v1 reset draw order, the transition and the v1 controller are
 * pinned by the reference's own recorded v1 run (gpu-d1/results/learning-v1-tests.log:1-3,
 * tests/test_v1_reference_run.py).
 */
#include "d1_oracle.h"
#include <stddef.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define W O_W
#define H O_H
#define N O_N

static inline int imin(int a, int b) { return a < b ? a : b; }
static inline int imax(int a, int b) { return a > b ? a : b; }
static inline int iabs(int a) { return a < 0 ? -a : a; }
/* gpu-d1/src/sim.h:14 */
static inline int cheb(int a, int b) { return imax(iabs(a % W - b % W), iabs(a / W - b / W)); }
/* gpu-d1/src/sim.h:201-206: N, E, S, W, NE, SE, SW, NW */
static const int DX[8] = {0, 1, 0, -1, 1, 1, -1, -1};
static const int DY[8] = {-1, 0, 1, 0, -1, 1, 1, -1};
static inline int neighbor(int p, int d) {
    int x = p % W + DX[d], y = p / W + DY[d];
    return x >= 0 && x < W && y >= 0 && y < H ? y * W + x : -1;
}

/* ------------------------------------------------------------------ RNG */
/* splitmix64 finaliser, gpu-d1/src/sim.h:15-20 */
uint64_t o_mix(uint64_t x) {
    x += 0x9e3779b97f4a7c15ULL;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ULL;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebULL;
    return x ^ (x >> 31);
}
/* Philox4x32-10 (Salmon et al., SC'11): multipliers 0xD2511F53/0xCD9E8D57,
 * Weyl key increments 0x9E3779B9/0xBB67AE85. */
void o_philox(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; r++) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n1 = (uint32_t)p1;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1, n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}
/* PCG32 XSH-RR step, gpu-d1/src/sim.h:23-28; counter mode: draw k of stream
 * (t, env, domain) is word k%4 of Philox(ctr={k/4, t, env, domain}, key=seed). */
static uint32_t rng_next(ORng *g) {
    if (g->mode == 0) {
        uint64_t old = g->state;
        g->state = old * 6364136223846793005ULL + (g->inc | 1);
        uint32_t x = (uint32_t)(((old >> 18) ^ old) >> 27), r = (uint32_t)(old >> 59);
        return (x >> r) | (x << ((-r) & 31));
    }
    uint32_t ctr[4] = {g->k >> 2, g->t, g->env, g->domain}, key[2] = {g->key0, g->key1}, o[4];
    o_philox(ctr, key, o);
    return o[g->k++ & 3];
}
/* gpu-d1/src/sim.h:29-35 */
static void pcg_seed(ORng *g, uint64_t s, uint64_t seq) {
    g->mode = 0;
    g->state = 0;
    g->inc = (seq << 1) | 1;
    rng_next(g);
    g->state += s;
    rng_next(g);
}
static void ctr_stream(ORng *g, uint64_t seed, uint32_t env, uint32_t t, uint32_t domain) {
    memset(g, 0, sizeof *g);
    g->mode = 1;
    g->key0 = (uint32_t)seed;
    g->key1 = (uint32_t)(seed >> 32);
    g->env = env;
    g->t = t;
    g->domain = domain;
}
/* Lemire bounded draw with the (-b)%b rejection threshold, gpu-d1/src/sim.h:36-51 */
static int rng_r(ORng *g, int bound) {
    if (bound <= 1) return 0;
    uint32_t x = rng_next(g);
    uint64_t m = (uint64_t)x * (uint32_t)bound;
    uint32_t low = (uint32_t)m;
    if (low < (uint32_t)bound) {
        uint32_t t = (uint32_t)(-(uint32_t)bound) % (uint32_t)bound;
        while (low < t) {
            x = rng_next(g);
            m = (uint64_t)x * (uint32_t)bound;
            low = (uint32_t)m;
        }
    }
    return (int)(m >> 32);
}
/* gpu-d1/src/sim.h:52-55 (both draws happen, left to right) */
static int rng_avg(ORng *g, int n) {
    int a = rng_r(g, n);
    return (a + rng_r(g, n + 1)) / 2;
}
/* gpu-d1/src/sim.h:56-59: draws only when n % d != 0 */
static int rng_round(ORng *g, int n, int d) {
    int rem = n % d;
    return n / d + (rem && rng_r(g, d) < rem);
}

/* Exported for the learn-task restatement (oracle/learn_oracle.c). */
uint32_t o_rng_next(ORng *g) { return rng_next(g); }
int o_rng_r(ORng *g, int bound) { return rng_r(g, bound); }
int o_rng_avg(ORng *g, int n) { return rng_avg(g, n); }
int o_rng_round(ORng *g, int n, int d) { return rng_round(g, n, d); }
void o_pcg_seed(ORng *g, uint64_t s, uint64_t seq) { pcg_seed(g, s, seq); }

void o_rng_ops(int mode, uint64_t seed, uint64_t seq, int nops, const int32_t *ops,
               const int32_t *args, int32_t *results, uint64_t *final_state) {
    ORng g;
    if (mode == 0) pcg_seed(&g, seed, seq);
    else ctr_stream(&g, seed, (uint32_t)seq, 0, 0);
    for (int i = 0; i < nops; i++) {
        switch (ops[i]) {
        case 0: results[i] = (int32_t)rng_next(&g); break;
        case 1: results[i] = rng_r(&g, args[i]); break;
        case 2: results[i] = rng_avg(&g, args[i]); break;
        default: results[i] = rng_round(&g, args[i] >> 8, args[i] & 255); break;
        }
    }
    final_state[0] = mode == 0 ? g.state : g.k;
}

/* ------------------------------------------------------------------ LOS */
static int g_nrays;
static int8_t g_ex[512], g_ey[512];
static uint64_t g_mask[512];

void o_set_rays(int nrays, const int8_t *ends_xy, const uint64_t *masks) {
    g_nrays = nrays > 512 ? 512 : nrays;
    for (int i = 0; i < g_nrays; i++) {
        g_ex[i] = ends_xy[2 * i];
        g_ey[i] = ends_xy[2 * i + 1];
        g_mask[i] = masks[i];
    }
}
/* Opaque inside-blocker set of one quadrant: blocker j = (j%8, j/8), opaque when
 * in bounds and not floor (gpu-d1/scripts/compile_fixture.py:35-39). */
static uint64_t quadrant_opaque(const uint8_t *floor, int px, int py, int sx, int sy) {
    uint64_t opq = 0;
    for (int j = 0; j < 64; j++) {
        int qx = px + sx * (j % 8), qy = py + sy * (j / 8);
        if (qx >= 0 && qx < W && qy >= 0 && qy < H && !floor[qy * W + qx]) opq |= 1ULL << j;
    }
    return opq;
}
/* The full 17x17 bitset of gpu-d1/scripts/compile_fixture.py:31-48 (bit (dy+8)*17+dx+8);
 * endpoints must be inside blockers, i.e. x, y < 8. */
void o_los_bitset(const uint8_t *floor, int origin, uint32_t out[10]) {
    static const int SX[4] = {1, -1, -1, 1}, SY[4] = {1, 1, -1, -1};
    int px = origin % W, py = origin / W;
    memset(out, 0, 40);
    out[144 / 32] |= 1u << (144 % 32);
    for (int q = 0; q < 4; q++) {
        uint64_t dead = quadrant_opaque(floor, px, py, SX[q], SY[q]);
        for (int i = 0; i < g_nrays; i++) {
            int x = g_ex[i], y = g_ey[i], qx = px + SX[q] * x, qy = py + SY[q] * y;
            if (!(g_mask[i] & dead) && qx >= 0 && qx < W && qy >= 0 && qy < H && x < 8 && y < 8) {
                int bit = (SY[q] * y + 8) * 17 + SX[q] * x + 8;
                out[bit / 32] |= 1u << (bit % 32);
            }
        }
    }
}
/* Point query used by the rules: target within `radius` (Chebyshev) and some
 * unblocked ray of a sign-compatible quadrant ends on it
 * (in_view / monster_detects_player, gpu-d1/branches/d1-stairs-v2/src/learn.cu:192-207). */
int o_los(const uint8_t *floor, int origin, int target, int radius) {
    static const int SX[4] = {1, -1, -1, 1}, SY[4] = {1, 1, -1, -1};
    if (target < 0 || target >= N) return 0;
    int px = origin % W, py = origin / W;
    int dx = target % W - px, dy = target / W - py;
    if (iabs(dx) > radius || iabs(dy) > radius) return 0;
    if (!dx && !dy) return 1;
    int ax = iabs(dx), ay = iabs(dy);
    if (ax > 7 || ay > 7) return 0;
    for (int q = 0; q < 4; q++) {
        if ((dx && (dx > 0) != (SX[q] > 0)) || (dy && (dy > 0) != (SY[q] > 0))) continue;
        uint64_t dead = quadrant_opaque(floor, px, py, SX[q], SY[q]);
        for (int i = 0; i < g_nrays; i++)
            if (g_ex[i] == ax && g_ey[i] == ay && !(g_mask[i] & dead)) return 1;
    }
    return 0;
}

/* ------------------------------------------------------------------ level generator */
/* Build-owned spec (the reference loads native Crawl exports instead). The
 * interior is split into 3x3 sectors of 26x22 cells (x0 = 1+26c, y0 = 1+22r);
 * n = 6 + U{0..3} sectors are chosen by a partial Fisher-Yates shuffle of 0..8
 * (swap i with i + U{0..8-i}); in shuffle order each chosen sector gets one room,
 * w = 4 + U{0..8}, h = 3 + U{0..5}, x = x0 + U{0..26-w}, y = y0 + U{0..22-h}; then
 * consecutive rooms are joined by an L-shaped corridor between their centres
 * (x + w/2, y + h/2), vertical leg first when a draw U{0,1} is 1. Every level is
 * connected, never touches the border, and has at least 72 floor cells. Counter
 * stream (seed, env, t=0, domain 1); the draw count is fixed by n. */
void o_level_generate(uint64_t seed, uint32_t env, uint8_t *floor) {
    ORng g;
    ctr_stream(&g, seed, env, 0, 1);
    memset(floor, 0, N);
    int n = 6 + rng_r(&g, 4);
    int order[9] = {0, 1, 2, 3, 4, 5, 6, 7, 8};
    for (int i = 0; i < n; i++) {
        int j = i + rng_r(&g, 9 - i), tmp = order[i];
        order[i] = order[j];
        order[j] = tmp;
    }
    int rx[9], ry[9], rw[9], rh[9];
    for (int i = 0; i < n; i++) {
        int x0 = 1 + 26 * (order[i] % 3), y0 = 1 + 22 * (order[i] / 3);
        int w = 4 + rng_r(&g, 9), h = 3 + rng_r(&g, 6);
        rx[i] = x0 + rng_r(&g, 27 - w);
        ry[i] = y0 + rng_r(&g, 23 - h);
        rw[i] = w;
        rh[i] = h;
    }
    for (int j = 0; j < n; j++)
        for (int y = ry[j]; y < ry[j] + rh[j]; y++)
            for (int x = rx[j]; x < rx[j] + rw[j]; x++) floor[y * W + x] = 1;
    for (int j = 1; j < n; j++) {
        int ax = rx[j - 1] + rw[j - 1] / 2, ay = ry[j - 1] + rh[j - 1] / 2;
        int bx = rx[j] + rw[j] / 2, by = ry[j] + rh[j] / 2;
        int vertical_first = rng_r(&g, 2);
        int cy = vertical_first ? by : ay, cx = vertical_first ? ax : bx;
        for (int x = imin(ax, bx); x <= imax(ax, bx); x++) floor[cy * W + x] = 1;
        for (int y = imin(ay, by); y <= imax(ay, by); y++) floor[y * W + cx] = 1;
    }
}

/* ------------------------------------------------------------------ rules */
static inline int floor_at(const OState *s, int p) { return p >= 0 && p < N && s->floor[p]; }
/* Player view: the 17x17 LOS bitset of the player's cell, memoised per position
 * (the reference reads the same bitset from its per-map LOS table). */
static int in_view(const OState *s, int p) {
    if (p < 0 || p >= N) return 0;
    int dx = p % W - s->player % W, dy = p / W - s->player / W;
    if (iabs(dx) > 7 || iabs(dy) > 7) return 0;
    OState *m = (OState *)s;
    if (m->vis_origin != s->player) { o_los_bitset(s->floor, s->player, m->vis); m->vis_origin = s->player; }
    int bit = (dy + 8) * 17 + dx + 8;
    return (s->vis[bit / 32] >> (bit % 32)) & 1;
}
static inline int seen_at(const OState *s, int p) { return s->viewed[p] && s->floor[p]; }
static const D1Kind *kind_of(const OState *s, const D1Config *c, int id) { return &c->kinds[s->kind[id]]; }

/* gpu-d1/branches/d1-stairs-v2/src/learn.cu:298-333 (MARK_WALLS; seen = viewed floor) */
static int reveal(OState *s) {
    int fresh = 0, px = s->player % W, py = s->player / W;
    for (int y = -7; y <= 7; y++)
        for (int x = -7; x <= 7; x++) {
            int qx = px + x, qy = py + y;
            if (qx < 0 || qx >= W || qy < 0 || qy >= H) continue;
            int p = qy * W + qx;
            if (!in_view(s, p)) continue;
            if (!s->viewed[p]) {
                s->viewed[p] = 1;
                if (s->floor[p]) fresh++;
            }
        }
    s->floor_seen += fresh;
    return fresh;
}
static int stair_index(const OState *s) {
    for (int k = 0; k < 3; k++) if (s->stairs[k] >= 0 && s->player == s->stairs[k]) return k + 1;
    return 0;
}
static int known_stairs(const OState *s) {
    int n = 0;
    for (int k = 0; k < 3; k++) n += s->stairs[k] >= 0 && seen_at(s, s->stairs[k]);
    return n;
}
static int visible_awake(const OState *s, const D1Config *c) {
    for (int i = 0; i < c->count; i++)
        if (s->mhp[i] > 0 && s->awake[i] && in_view(s, s->pos[i])) return 1;
    return 0;
}

/* Planted mistakes for the tests that show a fixture bites (0 = none, the faithful rules):
 * 1 a monster's energy drawn before its cell at reset, 2 the v1 controller's HP and
 * distance ties kept by the later candidate, 3 the player's melee damage 1 + r(5);
 * in the stairs reservoir: 4 drawn from the play stream instead of a copy, 5 stairs more
 * than 12 (not at least 12) from the player, 6 the spacing checked against all earlier
 * stairs but the last, 7 the draw bound counting every cell of the list, not the
 * eligible ones. */
static int planted;
void o_plant(int which) { planted = which; }

/* gpu-d1/branches/d1-stairs-v2/src/learn.cu:351-446 with the v1 roster
 * (gpu-d1/src/learn.cu:305-314); roster_mode 1 and awake_pct are build extensions
 * whose draws follow the energy draw. Clumped/ogre placement is not modelled. */
static void reset(OState *s, const D1Config *c) {
    static const int MHP[6] = {8, 10, 12, 16, 12, 10};
    ORng *g = &s->rng;
    for (int p = 0; p < N; p++) s->occ[p] = -1;
    s->player = s->cells[rng_r(g, s->ncells)];
    s->hp = c->hp; s->regen = 0; s->blocks = 0;
    s->ticks = 0; s->decisions = 0; s->killed = 0; s->floor_seen = 0;
    for (int i = 0; i < c->count; i++) {
        int p, tries = 0, early = planted == 1 ? rng_r(g, 10) : -1;
        do { p = s->cells[rng_r(g, s->ncells)]; } while ((p == s->player || s->occ[p] >= 0) && ++tries < 65536);
        /* The reference retries without bound; the cap (never reached with >= 72 cells
         * and <= 64 monsters) bounds the GPU loop, falling back to the first free cell. */
        if (p == s->player || s->occ[p] >= 0)
            for (int j = 0; j < s->ncells; j++) { p = s->cells[j]; if (p != s->player && s->occ[p] < 0) break; }
        s->pos[i] = (int16_t)p;
        s->occ[p] = (int16_t)i;
        if (c->roster_mode == 0) { s->kind[i] = (uint8_t)(i % 6); s->mhp[i] = (int16_t)MHP[i % 6]; }
        s->energy[i] = (int16_t)(70 + (early >= 0 ? early : rng_r(g, 10)));
        if (c->roster_mode == 1) {
            s->kind[i] = (uint8_t)rng_r(g, 6);
            s->mhp[i] = (int16_t)(c->hp_lo + rng_r(g, c->hp_hi - c->hp_lo + 1));
        }
        s->awake[i] = c->awake_pct >= 100 ? 1 : c->awake_pct <= 0 ? 0 : rng_r(g, 100) < c->awake_pct;
    }
    memset(s->viewed, 0, N);
    /* Stairs from a copy of the RNG (reservoir choice over the cell list). */
    ORng copy = *g, *stair = planted == 4 ? g : &copy;
    s->first_stair_tick = -1;
    for (int k = 0; k < 3; k++) {
        int selected = -1, count = 0;
        if (k < c->stairs)
            for (int j = 0; j < s->ncells; j++) {
                int p = s->cells[j];
                int eligible = cheb(p, s->player) >= (planted == 5 ? 13 : 12) && s->occ[p] < 0;
                for (int q = 0; q < k - (planted == 6); q++) eligible &= cheb(p, s->stairs[q]) >= 8;
                if (eligible && rng_r(stair, planted == 7 ? j + 1 : ++count) == 0) selected = p;
            }
        s->stairs[k] = selected;
    }
    reveal(s); /* the initial view earns no reward */
}

/* ------------------------------------------------------------------ monster rules (shared) */
static int m_kind(const OMonsters *m, int id, int field) {
    return m->kinds[4 * (m->kind_of ? m->kind_of[id] : id % 6) + field];
}
/* gpu-d1/src/sim.h:130-163: to-hit against EV (probabilistically rounded, averaged),
 * 5% automatic hit or miss, shield block against bypass while blocks < limit, damage
 * 1 + r(damage) minus max(r(ac + 1), min(gdr * damage / 100, ac rounded by halves)) with
 * the GDR table entry of a second, independent AC rounding. */
void o_m_attack(OMonsters *m, int id) {
    ORng *r = m->rng;
    int hit = rng_r(r, m_kind(m, id, 2) + 1);
    int ev = rng_round(r, m->ev100, 100);
    ev = rng_avg(r, 2 * ev);
    int margin = hit - ev;
    if (rng_r(r, 100) < 5) margin = (rng_r(r, 2) ? 1 : -1) * 1000;
    int bypass = rng_r(r, m_kind(m, id, 3));
    int sh = rng_round(r, m->sh100, 100);
    int block = rng_avg(r, sh * 2) / 3 - 1;
    if (block >= bypass && *m->blocks < m->shield_limit) { (*m->blocks)++; return; }
    if (margin < 0) return;
    int dmg = m_kind(m, id, 1);
    int damage = 1 + rng_r(r, dmg);
    int ac = rng_round(r, m->ac100, 100);
    int gac = rng_round(r, m->ac100, 100);
    int gdr = gac - m->ac100 / 100 ? m->gdr1 : m->gdr0;
    int saved = rng_r(r, ac + 1);
    int half = rng_round(r, ac, 2);
    saved = imax(saved, imin(gdr * dmg / 100, half));
    *m->hp -= imax(0, damage - saved);
}
static int m_passable(const OMonsters *m, int q) {
    return q >= 0 && m->floor[q] && q != m->player && m->occ[q] < 0;
}
/* gpu-d1/src/sim.h:207-253: greedy descent of the distance field, cardinals then
 * diagonals from a rotation r(4); equal improvements replace the choice with probability
 * 1/ties; when stuck (and repair is on), the first step of a 24-node breadth-first search
 * towards any lower-distance cell. */
int o_m_choose_move(OMonsters *m, const uint16_t *dist, int id) {
    int p = m->pos[id], best = -1, bd = dist[p], ties = 0, rotation = rng_r(m->rng, 4);
    for (int z = 0; z < 8; z++) {
        int d = z < 4 ? (z + rotation) % 4 : 4 + (z + rotation) % 4;
        int q = neighbor(p, d);
        if (!m_passable(m, q)) continue;
        int dd = dist[q];
        if (dd < bd) { bd = dd; best = q; ties = 1; }
        else if (dd == bd && best >= 0 && rng_r(m->rng, ++ties) == 0) best = q;
    }
    if (best >= 0 || !m->repair) return best;
    int cells[24], first[24], len = 1;
    cells[0] = p;
    first[0] = -1;
    for (int head = 0; head < len; head++)
        for (int d = 0; d < 8; d++) {
            int q = neighbor(cells[head], d);
            if (!m_passable(m, q)) continue;
            int seen = 0;
            for (int j = 0; j < len; j++) if (cells[j] == q) { seen = 1; break; }
            if (seen) continue;
            int step = head == 0 ? q : first[head];
            if (dist[q] < dist[p]) return step;
            if (len < 24) { cells[len] = q; first[len] = step; len++; }
        }
    return -1;
}
/* gpu-d1/src/sim.h:165-174: the next actor is the monster with the most energy >= 80,
 * ties to the lowest id (the heap of :175-200 picks the same one). */
int o_m_scan(const int16_t *energy, int count) {
    int best = -1;
    for (int i = 0; i < count; i++)
        if (energy[i] >= 80 && (best < 0 || energy[i] > energy[best] || (energy[i] == energy[best] && i < best)))
            best = i;
    return best;
}
/* gpu-d1/src/sim.h:254-269: pay 10 energy, then melee when adjacent, else move (`dist`
 * is read only for a move). */
void o_m_act(OMonsters *m, const uint16_t *dist, int id) {
    m->energy[id] = (int16_t)(m->energy[id] - 10);
    if (cheb(m->pos[id], m->player) == 1) { o_m_attack(m, id); return; }
    int q = o_m_choose_move(m, dist, id);
    if (q >= 0) {
        m->occ[m->pos[id]] = -1;
        m->pos[id] = (int16_t)q;
        m->occ[q] = (int16_t)id;
    }
}
/* the env world's view */
static OMonsters env_monsters(OState *s, const D1Config *c) {
    OMonsters m = {&s->rng, &s->hp, &s->blocks, s->pos, s->energy, s->occ, s->floor, s->kind,
                   (const int32_t *)c->kinds, s->player, c->ac100, c->ev100, c->sh100, c->shield_limit,
                   c->repair, c->gdr[0], c->gdr[1]};
    return m;
}
/* Distance field from `source` over floor, 8-neighbour BFS (what the reference's all-pairs
 * table rows hold, gpu-d1/scripts/learn_env.py:31-39); 65535 = unreached. */
static void floor_field(const OState *s, int source, uint16_t *ds) {
    static __thread int16_t queue[N];
    for (int p = 0; p < N; p++) ds[p] = 65535;
    int head = 0, tail = 1;
    queue[0] = (int16_t)source;
    ds[source] = 0;
    while (head < tail) {
        int p = queue[head++];
        for (int d = 0; d < 8; d++) {
            int q = neighbor(p, d);
            if (q >= 0 && s->floor[q] && ds[q] == 65535) { ds[q] = (uint16_t)(ds[p] + 1); queue[tail++] = (int16_t)q; }
        }
    }
}
static void player_field(const OState *s, uint16_t *ds) { floor_field(s, s->player, ds); }
/* LOS-gated waking, gpu-d1/branches/d1-stairs-v2/src/learn.cu:201-207; the v1
 * rule is Chebyshev <= 6 alone (gpu-d1/src/learn.cu:555-559). */
static int detects(const OState *s, const D1Config *c, int origin) {
    if (cheb(origin, s->player) > 6) return 0;
    return c->wake_los ? o_los(s->floor, origin, s->player, 6) : 1;
}

/* One physical turn, gpu-d1/branches/d1-stairs-v2/src/learn.cu:684-827 (primitive
 * d: 0-7 move/bump, 8 wait, 18 descend). out8 = [reward, done, clear, killed, hp,
 * ticks, death, timeout]; *saw_awake mirrors the reference's out[41]. */
static void primitive(OState *s, const D1Config *c, int d, float *out8, int *saw_awake) {
    static __thread uint16_t dist[N];
    int milli = c->step_milli, have_dist = 0;
    s->blocks = 0;
    s->regen += c->regen;
    while (s->regen >= 100) { s->hp = imin(c->hp, s->hp + 1); s->regen -= 100; }
    if (d >= 0 && d < 8) {
        int p = neighbor(s->player, d);
        if (floor_at(s, p)) {
            int id = s->occ[p];
            if (id >= 0) {
                if (rng_r(&s->rng, 5) != 0) {
                    s->mhp[id] = (int16_t)(s->mhp[id] - (1 + rng_r(&s->rng, planted == 3 ? 5 : 4)));
                    if (s->mhp[id] <= 0) {
                        s->mhp[id] = 0; s->occ[p] = -1; s->energy[id] = -30000;
                        s->killed++;
                        milli += c->kill_milli;
                    }
                }
            } else s->player = p;
        }
    }
    milli += c->explore_milli * reveal(s);
    int awake_seen = visible_awake(s, c);
    int clear = (d == 18 && stair_index(s) > 0 && s->hp > 0) ||
                (c->clear_on_kill_all && s->killed == c->count);
    if (!clear) {
        for (int i = 0; i < c->count; i++)
            if (s->mhp[i] > 0 && !s->awake[i] && detects(s, c, s->pos[i])) { s->awake[i] = 1; s->energy[i] = 70; }
        for (int i = 0; i < c->count; i++)
            if (s->mhp[i] > 0 && !s->awake[i]) s->energy[i] = -30000;
        for (int i = 0; i < c->count; i++)
            if (s->mhp[i] > 0) s->energy[i] = (int16_t)(s->energy[i] + kind_of(s, c, i)->speed);
        OMonsters mon = env_monsters(s, c);
        while (s->hp > 0) {
            int id = o_m_scan(s->energy, c->count);
            if (id < 0) break;
            if (!have_dist && cheb(s->pos[id], s->player) != 1) { player_field(s, dist); have_dist = 1; }
            o_m_act(&mon, dist, id);
            if (in_view(s, s->pos[id]) && s->awake[id]) awake_seen = 1;
        }
    }
    s->ticks++;
    if (s->first_stair_tick < 0 && known_stairs(s) > 0) s->first_stair_tick = s->ticks;
    int death = s->hp <= 0, timeout = !clear && !death && s->ticks >= c->limit;
    if (clear) milli += c->clear_milli;
    if (death) milli -= c->death_milli;
    float reward = 0.001f * (float)milli;
    reward -= c->turn_cost;
    awake_seen = awake_seen || visible_awake(s, c);
    out8[0] = reward; out8[1] = (float)(clear || death || timeout); out8[2] = (float)clear;
    out8[3] = (float)s->killed; out8[4] = (float)imax(0, s->hp); out8[5] = (float)s->ticks;
    out8[6] = (float)death; out8[7] = (float)timeout;
    *saw_awake = awake_seen;
    if (clear || death || timeout) { s->episode++; reset(s, c); }
}

/* Joint action, gpu-d1/branches/d1-stairs-v2/src/learn.cu:852-875: MOVE 0-7,
 * ATTACK 8-15, WAIT 16, REST 17 (repeated waits), DESCEND 18; invalid -> one wait. */
static void transition(OState *s, const D1Config *c, int action, float *out) {
    int decisions = s->decisions + 1, invalid = 0;
    float total = 0.f, out8[8];
    for (;;) {
        int d = 8, saw;
        if (action >= 0 && action < 16) {
            int dir = action % 8, p = neighbor(s->player, dir);
            int enemy = p >= 0 && in_view(s, p) && s->occ[p] >= 0;
            int valid = action < 8 ? p >= 0 && (!s->viewed[p] || floor_at(s, p)) && !enemy : enemy;
            if (valid) d = dir; else invalid = 1;
        } else if (action == 17) invalid = s->hp >= c->hp || visible_awake(s, c) || c->regen <= 0;
        else if (action == 18) { if (stair_index(s) > 0) d = 18; else invalid = 1; }
        else if (action != 16) invalid = 1;
        primitive(s, c, d, out8, &saw);
        total += out8[0];
        if (out8[1] != 0.f || invalid || action != 17) break;
        if (saw || s->hp >= c->hp) break;
    }
    out[0] = total;
    for (int j = 1; j < 8; j++) out[j] = out8[j];
    if (out8[1] == 0.f) s->decisions = decisions;
}

/* ------------------------------------------------------------------ observation + hash */
/* 15x15x8 uint8, cell ((dy+7)*15+dx+7)*8 + channel:
 * 0 wall (out of bounds, or viewed non-floor), 1 floor (viewed floor), 2 visible,
 * 3 monster kind+1 (visible living), 4 monster HP (visible living, <=255),
 * 5 player HP (all cells), 6 remembered stair, 7 frontier anchor (seen floor with an
 * in-bounds unviewed neighbour, the FRONTIER_RING_MEMORY_WALLS rule of
 * gpu-d1/branches/d1-stairs-v2/src/learn.cu:269-280). */
void o_obs(const OState *s, const D1Config *c, uint8_t *o) {
    (void)c;
    int px = s->player % W, py = s->player / W, php = imin(imax(s->hp, 0), 255);
    for (int dy = -7; dy <= 7; dy++)
        for (int dx = -7; dx <= 7; dx++) {
            uint8_t *ch = o + ((dy + 7) * 15 + dx + 7) * 8;
            int x = px + dx, y = py + dy, inb = x >= 0 && x < W && y >= 0 && y < H, p = y * W + x;
            memset(ch, 0, 8);
            ch[5] = (uint8_t)php;
            if (!inb) { ch[0] = 1; continue; }
            ch[0] = s->viewed[p] && !s->floor[p];
            ch[1] = s->viewed[p] && s->floor[p];
            int vis = in_view(s, p);
            ch[2] = (uint8_t)vis;
            int id = s->occ[p];
            if (vis && id >= 0 && s->mhp[id] > 0) { ch[3] = (uint8_t)(s->kind[id] + 1); ch[4] = (uint8_t)imin(s->mhp[id], 255); }
            for (int k = 0; k < 3; k++) if (s->stairs[k] == p && seen_at(s, p)) ch[6] = 1;
            if (seen_at(s, p))
                for (int d = 0; d < 8; d++) {
                    int q = neighbor(p, d);
                    if (q >= 0 && !s->viewed[q]) { ch[7] = 1; break; }
                }
        }
}
static inline uint32_t fmix32(uint32_t h) {
    h ^= h >> 16; h *= 0x85ebca6bu; h ^= h >> 13; h *= 0xc2b2ae35u; h ^= h >> 16;
    return h;
}
static inline uint32_t term(uint32_t word, uint32_t index) { return fmix32(word ^ (index * 0x9E3779B9u)); }
/* State hash: sum mod 2^32 of fmix32(word ^ index*golden) over canonical words:
 * 0 player, 1 hp, 2 regen, 3 ticks, 4 killed, 5 decisions, 6 floor_seen, 7 episode,
 * 8/9 PCG state lo/hi (0 in counter mode), 10 step counter t, 11-13 stairs,
 * 14 first_stair_tick; 100+2i pos|hp<<16, 101+2i energy&0xffff|awake<<16|kind<<24;
 * 1000+3y+j viewed row y word j (80 bits, x-bit order). */
uint32_t o_hash(const OState *s, const D1Config *c) {
    uint32_t h = 0;
    uint32_t w[15] = {(uint32_t)s->player, (uint32_t)s->hp, (uint32_t)s->regen, (uint32_t)s->ticks,
                      (uint32_t)s->killed, (uint32_t)s->decisions, (uint32_t)s->floor_seen,
                      (uint32_t)s->episode, (uint32_t)s->rng.state * (s->rng.mode == 0),
                      (uint32_t)(s->rng.state >> 32) * (s->rng.mode == 0), s->t,
                      (uint32_t)s->stairs[0], (uint32_t)s->stairs[1], (uint32_t)s->stairs[2],
                      (uint32_t)s->first_stair_tick};
    for (uint32_t j = 0; j < 15; j++) h += term(w[j], j);
    for (int i = 0; i < c->count; i++) {
        h += term((uint16_t)s->pos[i] | (uint32_t)(uint16_t)s->mhp[i] << 16, 100 + 2 * i);
        h += term((uint16_t)s->energy[i] | (uint32_t)s->awake[i] << 16 | (uint32_t)s->kind[i] << 24, 101 + 2 * i);
    }
    for (int y = 0; y < H; y++)
        for (int j = 0; j < 3; j++) {
            uint32_t v = 0;
            for (int b = 0; b < 32 && 32 * j + b < W; b++) v |= (uint32_t)s->viewed[y * W + 32 * j + b] << b;
            h += term(v, 1000 + 3 * y + j);
        }
    return h;
}

/* ------------------------------------------------------------------ batch API */
int o_state_bytes(void) { return (int)sizeof(OState); }

/* Single-world hooks for the restated reference fixtures (tests/test_env_oracle_fixtures.py).
 * o_field_offset(k): byte offset of the k-th OState field in declaration order (k = 0..30),
 * sizeof(OState) for k = 31. */
int o_field_offset(int k) {
    static const int off[] = {
        (int)offsetof(OState, rng), (int)offsetof(OState, env_id), (int)offsetof(OState, t),
        (int)offsetof(OState, episode), (int)offsetof(OState, player), (int)offsetof(OState, hp),
        (int)offsetof(OState, regen), (int)offsetof(OState, blocks), (int)offsetof(OState, ticks),
        (int)offsetof(OState, killed), (int)offsetof(OState, decisions), (int)offsetof(OState, floor_seen),
        (int)offsetof(OState, first_stair_tick), (int)offsetof(OState, stairs), (int)offsetof(OState, ncells),
        (int)offsetof(OState, vis_origin), (int)offsetof(OState, vis), (int)offsetof(OState, pos),
        (int)offsetof(OState, mhp), (int)offsetof(OState, energy), (int)offsetof(OState, awake),
        (int)offsetof(OState, kind), (int)offsetof(OState, occ), (int)offsetof(OState, viewed),
        (int)offsetof(OState, floor), (int)offsetof(OState, cells), (int)offsetof(OState, rng.state),
        (int)offsetof(OState, rng.inc), (int)offsetof(OState, rng.mode), (int)offsetof(OState, rng.k),
        (int)offsetof(OState, rng.t), (int)sizeof(OState)};
    return k >= 0 && k < (int)(sizeof off / sizeof off[0]) ? off[k] : -1;
}
/* An empty world on a given map: every field zero, the byte floor and spawnable-cell masks
 * copied, occupancy cleared, no player view memoised, stairs absent. */
void o_world_map(OState *s, const uint8_t *floor, const uint8_t *cells) {
    memset(s, 0, sizeof *s);
    memcpy(s->floor, floor, N);
    for (int p = 0; p < N; p++) {
        s->occ[p] = -1;
        if (cells[p]) s->cells[s->ncells++] = (int16_t)p;
    }
    s->vis_origin = -1;
    s->first_stair_tick = -1;
    for (int k = 0; k < 3; k++) s->stairs[k] = -1;
}
void o_reset(OState *s, const D1Config *c) { reset(s, c); }
int o_reveal(OState *s) { return reveal(s); }
void o_transition(OState *s, const D1Config *c, int action, float *out8) { transition(s, c, action, out8); }

static void init_one(OState *s, uint32_t env, const D1Config *c, const uint8_t *floor,
                     const uint8_t *cells, uint64_t seed) {
    memset(s, 0, sizeof *s);
    s->vis_origin = -1;
    s->env_id = env;
    if (c->level_mode == 1) o_level_generate(seed, env, s->floor);
    else memcpy(s->floor, floor, N);
    s->ncells = 0;
    for (int p = 0; p < N; p++)
        if (c->level_mode == 1 ? s->floor[p] : cells[p]) s->cells[s->ncells++] = (int16_t)p;
    if (c->rng_mode == 0) pcg_seed(&s->rng, o_mix(seed + env), (uint64_t)env + 1);
    else ctr_stream(&s->rng, seed, env, 0, 2);
    s->t = 0;
    reset(s, c);
}
static void begin_step(OState *s) {
    if (s->rng.mode == 1) { s->rng.t = s->t; s->rng.k = 0; s->rng.domain = 0; }
}
int o_init(OState *st, int n, const D1Config *c, const uint8_t *floor, const uint8_t *cells,
           uint64_t seed, uint8_t *obs, uint32_t *hash, int threads) {
    if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int i = 0; i < n; i++) {
        init_one(&st[i], (uint32_t)i, c, floor, cells, seed);
        if (obs) o_obs(&st[i], c, obs + (size_t)i * 1800);
        if (hash) hash[i] = o_hash(&st[i], c);
    }
    return 0;
}
int o_step(OState *st, int n, const D1Config *c, const int64_t *actions, uint8_t *obs,
           float *out, uint32_t *hash, const uint8_t *active, int threads) {
    if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int i = 0; i < n; i++) {
        if (active && !active[i]) continue;
        OState *s = &st[i];
        begin_step(s);
        transition(s, c, (int)actions[i], out + (size_t)i * 8);
        s->t++;
        if (obs) o_obs(s, c, obs + (size_t)i * 1800);
        if (hash) hash[i] = o_hash(s, c);
    }
    return 0;
}

/* ------------------------------------------------------------------ wait benchmark */
/* The reference's monster-wait workload (gpu-d1/src/sim.h:93-122,270-295 driven as
 * in gpu-d1/src/bench.cu:151-184): a stationary player on map 1057, monsters at the
 * fixture spawn list, all awake, the static distance field; trace[k] is a digest
 * of the world after step k. Used only to pin the rule core against sim.h. */
typedef struct WaitWorld {
    ORng rng;
    int32_t hp, regen, blocks, fixture, episode;
    int16_t pos[64], energy[64], occ[N];
} WaitWorld;
static void wait_reset(WaitWorld *w, int count, const int32_t *cfg, const int16_t *starts, int first) {
    if (!first) for (int i = 0; i < count; i++) w->occ[w->pos[i]] = -1;
    w->hp = cfg[2]; w->regen = 0; w->blocks = 0;
    for (int i = 0; i < count; i++) {
        int p = starts[w->fixture * 64 + i];
        w->pos[i] = (int16_t)p; w->occ[p] = (int16_t)i;
        w->energy[i] = (int16_t)(70 + rng_r(&w->rng, 10));
    }
    if (!first) w->episode++;
}
static void wait_step(WaitWorld *w, int count, int heap_order, const int32_t *cfg, const int32_t *kinds,
                      const uint8_t *floor, const uint16_t *dist, const int16_t *starts) {
    if (w->hp <= 0) wait_reset(w, count, cfg, starts, 0);
    w->blocks = 0;
    w->regen += cfg[7];
    while (w->regen >= 100) { w->hp = imin(cfg[2], w->hp + 1); w->regen -= 100; }
    for (int i = 0; i < count; i++) w->energy[i] = (int16_t)(w->energy[i] + kinds[4 * (i % 6)]);
    /* The heap and the scan pick the same actor (gpu-d1/src/bench.cu:363-371); the
     * oracle always scans, `heap_order` only selects which reference run it mirrors. */
    (void)heap_order;
    OMonsters m = {&w->rng, &w->hp, &w->blocks, w->pos, w->energy, w->occ, floor, NULL, kinds,
                   cfg[1], cfg[3], cfg[4], cfg[5], cfg[6], cfg[8], cfg[9], cfg[10]};
    while (w->hp > 0) {
        int id = o_m_scan(w->energy, count);
        if (id < 0) break;
        o_m_act(&m, dist, id);
    }
}
static uint32_t wait_digest(const WaitWorld *w, int count) {
    uint32_t h = term((uint32_t)w->hp, 0) + term((uint32_t)w->regen, 1) + term((uint32_t)w->blocks, 2) +
                 term((uint32_t)w->episode, 3) + term((uint32_t)w->rng.state, 4) +
                 term((uint32_t)(w->rng.state >> 32), 5);
    for (int i = 0; i < count; i++)
        h += term((uint16_t)w->pos[i] | (uint32_t)(uint16_t)w->energy[i] << 16, 100 + i);
    return h;
}
int o_wait_run(int count, int steps, int heap, int scenario_fixture, uint64_t seed, uint32_t world,
               const uint8_t *floor, const uint16_t *dist, const int16_t *starts,
               const int32_t *cfg, const int32_t *kinds, int32_t prewarm, int32_t *trace) {
    static __thread WaitWorld w;
    memset(&w, 0, sizeof w);
    for (int p = 0; p < N; p++) w.occ[p] = -1;
    pcg_seed(&w.rng, o_mix(seed + world), (uint64_t)world + 1);
    w.fixture = scenario_fixture;
    wait_reset(&w, count, cfg, starts, 1);
    for (int k = 0; k < prewarm; k++) wait_step(&w, count, heap, cfg, kinds, floor, dist, starts);
    for (int k = 0; k < steps; k++) {
        wait_step(&w, count, heap, cfg, kinds, floor, dist, starts);
        trace[k] = (int32_t)wait_digest(&w, count);
    }
    return 0;
}

/* ------------------------------------------------------------------ heuristic */
/* Deterministic controller for test action streams (build-owned, simplified from
 * gpu-d1/branches/d1-stairs-v2/src/learn.cu:876-888): descend on a stair, else attack
 * the weakest visible adjacent monster, else step along the true distance field
 * toward the nearest living monster, else wait. */
/* gpu-d1/src/learn.cu:599-621, the v1 task's pursuit controller and the action stream of its
 * parity run (gpu-d1/scripts/test_learning.py:48). Returns a v1 action: direction 0-7 (move,
 * or melee when the cell holds a monster) or 8 (wait). The living adjacent monster with the
 * least HP first, a strictly lower HP replacing the choice, so ties keep the earlier direction;
 * else the living monster nearest to the player by floor distance (strictly nearer replaces:
 * ties keep the lowest id), then the neighbouring floor cell with the least distance to that
 * monster's cell among those strictly closer than the player's own (earlier directions win
 * ties); 8 when no monster lives or no neighbour is closer. */
int o_heuristic_v1(OState *s, const D1Config *c) {
    static __thread uint16_t dist[N];
    int best = -1, bhp = 10000;
    for (int d = 0; d < 8; d++) {
        int p = neighbor(s->player, d);
        if (p >= 0 && s->occ[p] >= 0 && (s->mhp[s->occ[p]] < bhp || (planted == 2 && s->mhp[s->occ[p]] == bhp))) {
            bhp = s->mhp[s->occ[p]]; best = d;
        }
    }
    if (best >= 0) return best;
    player_field(s, dist);
    int target = -1, bd = 65535;
    for (int i = 0; i < c->count; i++)
        if (s->mhp[i] > 0 && (dist[s->pos[i]] < bd || (planted == 2 && dist[s->pos[i]] == bd))) {
            bd = dist[s->pos[i]]; target = s->pos[i];
        }
    if (target < 0) return 8;
    floor_field(s, target, dist);
    const int own = dist[s->player];
    bd = own;
    best = 8;
    for (int d = 0; d < 8; d++) {
        int p = neighbor(s->player, d);
        if (floor_at(s, p) && (dist[p] < bd || (planted == 2 && dist[p] == bd && dist[p] < own))) { bd = dist[p]; best = d; }
    }
    return best;
}
int o_heuristic(OState *s, const D1Config *c) {
    static __thread uint16_t dist[N];
    if (stair_index(s) > 0) return 18;
    int best = -1, bhp = 100000;
    for (int d = 0; d < 8; d++) {
        int p = neighbor(s->player, d);
        if (p < 0) continue;
        int id = s->occ[p];
        if (id >= 0 && s->mhp[id] > 0 && in_view(s, p) && s->mhp[id] < bhp) { bhp = s->mhp[id]; best = d; }
    }
    if (best >= 0) return 8 + best;
    player_field(s, dist);
    int target = -1, bd = 65535;
    for (int i = 0; i < c->count; i++)
        if (s->mhp[i] > 0 && dist[s->pos[i]] < bd) { bd = dist[s->pos[i]]; target = s->pos[i]; }
    if (target < 0) return 16;
    /* walk back from the target along decreasing distance to the player's neighbour */
    int p = target;
    while (dist[p] > 1) {
        int prev = -1;
        for (int d = 0; d < 8; d++) {
            int q = neighbor(p, d);
            if (q >= 0 && s->floor[q] && dist[q] + 1 == dist[p]) { prev = q; break; }
        }
        if (prev < 0) return 16;
        p = prev;
    }
    for (int d = 0; d < 8; d++) if (neighbor(s->player, d) == p) return d;
    return 16;
}
