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

#ifdef __cplusplus
extern "C" {
#endif
uint64_t o_mix(uint64_t x);
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
/* single-function hooks compared against the reference's sim.h */
void o_rng_ops(int mode, uint64_t seed, uint64_t seq, int nops, const int32_t *ops,
               const int32_t *args, int32_t *results, uint64_t *final_state);
int o_wait_run(int count, int steps, int heap, int scenario_fixture, uint64_t seed, uint32_t world,
               const uint8_t *floor, const uint16_t *dist, const int16_t *starts,
               const int32_t *cfg11, const int32_t *kinds24, int32_t prewarm, int32_t *trace);
#ifdef __cplusplus
}
#endif
#endif
