/* d1learn: drop-in C ABI for the reference's d1-stairs-v2 task library.
 *
 * Same exported names, argument order and meaning as the reference's `learn_*`
 * exports (gpu-d1/branches/d1-stairs-v2/src/learn.cu:913-946), so its ctypes
 * wrapper (gpu-d1/branches/d1-stairs-v2/scripts/learn_env_ring_multi.py:26-46,
 * 63-120) binds this library unchanged. The task is the one its asset build
 * compiles (gpu-d1/branches/d1-stairs-v2/scripts/assets.py:5): 24 ordinary enemies,
 * LOS waking, remembered 15x15 terrain, 64-cell ring, frontier pointer + route cue,
 * three hidden stairs and DESCEND, +1 for descent and -1e-5 per physical turn,
 * 2,048-turn deadline passed as `limit`. Two libraries are built from one source,
 * as the reference builds two: CLUMP_MODE 0 (libd1learn_clump0.so) and 1
 * (libd1learn_clump1.so, a third of resets place the enemies in clumps of three).
 *
 * Differences from the reference, all at the boundary's edges:
 *   - `state` rows are this library's own compact layout (learn_state_bytes() bytes
 *     per env; rows stay per-env so `state[~active]` slicing keeps working);
 *   - `gpu` must be non-zero: there is no host path (returns D1L_E_HOST);
 *   - a bad argument or configuration returns a negative code instead of a device
 *     assert (the reference asserts count == 24 in reset, learn.cu:352).
 * All launches are asynchronous on `stream` (a hipStream_t; 0 = null stream).
 */
#ifndef D1LEARN_H
#define D1LEARN_H
#include <stdint.h>
#ifndef __cplusplus
#include <stdbool.h>
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define D1L_OBS 1015     /* learn.cu:101-112 */
#define D1L_ACTIONS 19   /* learn.cu:80: MOVE 0-7, ATTACK 8-15, WAIT 16, REST 17, DESCEND 18 */
#define D1L_OUT 45       /* learn.cu:80 */
#define D1L_ENEMIES 40   /* observation slots, LEARN_ENEMIES=40 in assets.py:5 */
#define D1L_REQUIRED 24  /* enemies per episode, learn.cu:39 */

#define D1L_E_ARG (-1)
#define D1L_E_CONFIG (-2)
#define D1L_E_HOST (-3)

/* sim::Kind / sim::Config (gpu-d1/src/sim.h:61-67): 35 ints, 140 bytes. */
typedef struct D1LKind {
    int32_t speed, damage, tohit, bypass;
} D1LKind;
typedef struct D1LConfig {
    int32_t count, player, hp, ac100, ev100, sh100, shield_limit, regen, repair, gdr[2];
    D1LKind kinds[6];
} D1LConfig;

/* learn::Tables with MULTI_MAP (gpu-d1/branches/d1-stairs-v2/src/learn.cu:143-153;
 * ctypes layout learn_env_ring_multi.py:11-17). Device pointers. Per map m:
 * floor[m*5600 + p], cells[m*5600 + j] (j < map_ncells[m]), los[(m*5600 + p)*10 + w].
 * `index`, `distance` and `distance_offsets` (the all-pairs floor BFS table) are
 * accepted and not read: the library computes the same player-distance rows by BFS
 * over floor on the fly. `ncells` is unused with MULTI_MAP, as in the reference. */
typedef struct D1LTables {
    const uint8_t *floor;
    const int16_t *cells, *index;
    const uint16_t *distance;
    int32_t ncells;
    const int32_t *map_ncells, *distance_offsets;
    int32_t n_maps, map_filter;
    const uint32_t *los;
} D1LTables;

float learn_turn_cost(void);     /* learn.cu:913 */
float learn_return_gamma(void);  /* learn.cu:914 */
int learn_state_bytes(void);     /* learn.cu:915 */
int learn_obs_size(void);        /* learn.cu:916 */
int learn_action_size(void);     /* learn.cu:917 */
int learn_out_size(void);        /* learn.cu:918 */
int learn_config_bytes(void);    /* learn.cu:919 */

/* learn.cu:891-899,920-931: seed env i with PCG32(mix(seed+i), i+1), reset, observe.
 * map_filter -2 gives env i map i % n_maps for its first episode. */
int learn_init(void *state, int n, const D1LConfig *cfg, const D1LTables *tab, uint64_t seed, float *obs,
               float *mask, void *stream, int gpu);
/* learn.cu:932-936: one joint action per env (REST repeats internal turns); an action's
 * low 32 bits are taken as a signed int, as the reference's int parameter takes it. */
int learn_step(void *state, int n, const D1LConfig *cfg, const D1LTables *tab, const int64_t *actions, int limit,
               float *obs, float *mask, float *out, void *stream, int gpu);
/* learn.cu:937-941: envs with active[i] == false keep state, obs, mask and out. */
int learn_step_active(void *state, int n, const D1LConfig *cfg, const D1LTables *tab, const int64_t *actions,
                      int limit, float *obs, float *mask, float *out, const bool *active, void *stream, int gpu);
/* learn.cu:942-946: the deterministic stairs/attack/rest/engage/explore controller. */
int learn_heuristic(void *state, int n, const D1LConfig *cfg, const D1LTables *tab, int64_t *actions, void *stream,
                    int gpu);

#ifdef __cplusplus
}
#endif
#endif
