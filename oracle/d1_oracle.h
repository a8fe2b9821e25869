/* TEST INFRASTRUCTURE ONLY — CPU restatement of the reference D:1 rules.
 *
 * This oracle is the checker for the HIP library in dcss-auto_amd/csrc. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * the product path never links or calls it.
 */
#ifndef D1_ORACLE_H
#define D1_ORACLE_H
#include <stdint.h>
#include "../include/d1hip.h"

#define O_W 80
#define O_H 70
#define O_N 5600
#define O_MAXM 64

typedef struct ORng {
    uint64_t state, inc;                 /* PCG32 */
    uint32_t key0, key1, t, env, domain, k; /* Philox4x32-10 counter stream */
    int32_t mode;                        /* 0 pcg, 1 counter */
    int32_t pad;
} ORng;

/* One world, array-of-structs like the reference's learn::State. */
typedef struct OState {
    ORng rng;
    uint32_t env_id, t;
    int32_t episode;
    int32_t player, hp, regen, blocks;
    int32_t ticks, killed, decisions, floor_seen, first_stair_tick;
    int32_t stairs[3];
    int32_t ncells;
    int32_t vis_origin;         /* memo: LOS bitset of the cell below (not state) */
    uint32_t vis[10];
    int16_t pos[O_MAXM], mhp[O_MAXM], energy[O_MAXM];
    uint8_t awake[O_MAXM], kind[O_MAXM];
    int16_t occ[O_N];
    uint8_t viewed[O_N];
    uint8_t floor[O_N];
    int16_t cells[O_N];
} OState;

/* One world of the d1-stairs-v2 learning task, the fields of the reference's
 * learn::State (gpu-d1/branches/d1-stairs-v2/src/learn.cu:113-142) that the task
 * with 24 enemies and no ogres reads. `error` records a reset that the reference
 * would stop with an assert (no clump anchor or stair cell). */
#define O_LE 40
typedef struct LState {
    ORng rng;
    int32_t map_id, player, hp, regen, blocks, ticks, killed, decisions, episode;
    int32_t next_slot, floor_seen, first_stair_tick, placement_clumped, frontier_count, error;
    int32_t stairs[3];
    int16_t pos[O_LE], energy[O_LE], mhp[O_LE], awake[O_LE], enemy_slot[O_LE];
    uint8_t encountered[O_LE];
    int16_t occ[O_N];
    uint8_t seen[O_N], viewed[O_N];
    int16_t frontier_cells[O_N], frontier_slot[O_N];
} LState;

/* The monster rules of gpu-d1/src/sim.h:130-269 (melee, scheduler, greedy move with the
 * 24-node repair search, act), written once for every world type of this oracle: the env
 * worlds (OState), the learning-task worlds (LState) and the wait-benchmark worlds all hand
 * the same functions a view of their fields, so the sim.h golden traces that pin these
 * functions through the wait worlds pin the code the other two run. */
typedef struct OMonsters {
    ORng *rng;
    int32_t *hp, *blocks;               /* the player's */
    int16_t *pos, *energy, *occ;        /* occ[5600]: monster id on the cell or -1 */
    const uint8_t *floor;               /* byte per cell, nonzero = floor */
    const uint8_t *kind_of;             /* kind index per monster, or NULL for id % 6 */
    const int32_t *kinds;               /* 6 x {speed, damage, tohit, bypass} */
    int32_t player, ac100, ev100, sh100, shield_limit, repair, gdr0, gdr1;
} OMonsters;

#ifdef __cplusplus
extern "C" {
#endif
int o_m_scan(const int16_t *energy, int count);                       /* sim.h:165-174 */
void o_m_attack(OMonsters *m, int id);                                /* sim.h:130-163 */
int o_m_choose_move(OMonsters *m, const uint16_t *dist, int id);      /* sim.h:207-253 */
void o_m_act(OMonsters *m, const uint16_t *dist, int id);             /* sim.h:254-269 */
uint64_t o_mix(uint64_t x);
uint32_t o_rng_next(ORng *g);
int o_rng_r(ORng *g, int bound);
int o_rng_avg(ORng *g, int n);
int o_rng_round(ORng *g, int n, int d);
void o_pcg_seed(ORng *g, uint64_t s, uint64_t seq);
void o_philox(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
void o_set_rays(int nrays, const int8_t *ends_xy, const uint64_t *masks);
void o_los_bitset(const uint8_t *floor, int origin, uint32_t out[10]);
int o_los(const uint8_t *floor, int origin, int target, int radius);
void o_level_generate(uint64_t seed, uint32_t env, uint8_t *floor);
int o_state_bytes(void);
int o_init(OState *st, int n, const D1Config *c, const uint8_t *floor, const uint8_t *cells,
           uint64_t seed, uint8_t *obs, uint32_t *hash, int threads);
int o_step(OState *st, int n, const D1Config *c, const int64_t *actions, uint8_t *obs,
           float *out, uint32_t *hash, const uint8_t *active, int threads);
void o_obs(const OState *s, const D1Config *c, uint8_t *obs);
uint32_t o_hash(const OState *s, const D1Config *c);
int o_heuristic(OState *s, const D1Config *c);
int o_heuristic_v1(OState *s, const D1Config *c);                      /* learn.cu:599-621 */
void o_plant(int which);   /* planted mistakes for tests (d1_oracle.c); 0 = the faithful rules */
void lo_plant(int which);  /* the same for the learning task's reset (learn_oracle.c) */
int o_field_offset(int k);
void o_world_map(OState *s, const uint8_t *floor, const uint8_t *cells);
void o_reset(OState *s, const D1Config *c);
int o_reveal(OState *s);
void o_transition(OState *s, const D1Config *c, int action, float *out8);
/* single-function hooks compared against the reference's sim.h */
void o_rng_ops(int mode, uint64_t seed, uint64_t seq, int nops, const int32_t *ops,
               const int32_t *args, int32_t *results, uint64_t *final_state);
int o_wait_run(int count, int steps, int heap, int scenario_fixture, uint64_t seed, uint32_t world,
               const uint8_t *floor, const uint16_t *dist, const int16_t *starts,
               const int32_t *cfg11, const int32_t *kinds24, int32_t prewarm, int32_t *trace);

/* learn-task restatement (oracle/learn_oracle.c); tables hold host pointers */
struct D1LConfig;
struct D1LTables;
int lo_state_bytes(void);
int lo_field_offset(int k);
int lo_init(LState *st, int n, const struct D1LConfig *c, const struct D1LTables *t, uint64_t seed, float *obs,
            float *mask, int clump, int threads);
int lo_step(LState *st, int n, const struct D1LConfig *c, const struct D1LTables *t, const int64_t *actions, int limit,
            float *obs, float *mask, float *out, const uint8_t *active, int clump, int threads);
int lo_heuristic(LState *st, int n, const struct D1LConfig *c, const struct D1LTables *t, int64_t *actions,
                 int threads);
void lo_reset(LState *s, const struct D1LConfig *c, const struct D1LTables *t, int clump);
int lo_reveal(LState *s, const struct D1LTables *t);
void lo_refresh_frontier(LState *s, const struct D1LTables *t, int p);
void lo_observe(LState *s, const struct D1LConfig *c, const struct D1LTables *t, float *obs, float *mask);
void lo_known_distances(const LState *s, const struct D1LTables *t, uint16_t *ds, int nearest_only);
int lo_route_first_step(int player, int target, const uint16_t *ds);
int lo_nearest_stair(const LState *s, const uint16_t *ds);
int lo_in_view(const LState *s, const struct D1LTables *t, int p);
void lo_transition(LState *s, const struct D1LConfig *c, const struct D1LTables *t, int action, int limit,
                   float *out, int clump);
int lo_heuristic_one(LState *s, const struct D1LConfig *c, const struct D1LTables *t);
void lo_distance_table(const uint8_t *floor, const int16_t *cells, int ncells, uint16_t *out);
void lo_los_table(const uint8_t *floor, uint32_t *out);
#ifdef __cplusplus
}
#endif
#endif
