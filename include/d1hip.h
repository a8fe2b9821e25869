/* d1hip — MI355X-native batched DCSS D:1 environment (C ABI).
 *
 * One call steps a batch of independent D:1 worlds on the GPU: the player's
 * semantic action (MOVE 0-7, ATTACK 8-15, WAIT 16, REST 17, DESCEND 18),
 * field-of-view reveal, LOS-gated monster waking, the monster turn loop
 * (energy scheduler, greedy pathing on a distance-from-player field, melee),
 * terminal checks with in-step auto-reset, the 15x15x8 uint8 egocentric
 * observation and a per-env 32-bit state hash.
 *
 * The entry points mirror the reference's `learn_*` C ABI
 * (gpu-d1/src/learn.cu:643-675, gpu-d1/branches/d1-stairs-v2/src/learn.cu:912-945):
 * size queries, init, step, step-with-active-mask. Differences, by design:
 *   - observations are uint8 [n, 15, 15, 8] (channel-last) instead of fp32 vectors;
 *   - the per-env state row also holds that env's level (floor + spawnable cells),
 *     so each env may carry its own generated level;
 *   - a 32-bit state hash per env is written on every call;
 *   - only the GPU path exists here (the reference's `gpu` flag selected a host
 *     loop; the CPU restatement used for verification lives outside this library).
 *
 * All pointers are device pointers except `cfg` and `tab`, which are host structs
 * copied by value into the launch. Calls are asynchronous on `stream` (a
 * hipStream_t; 0 = the null stream). Return value: 0 on success, a hipError_t
 * code for launch failures, or a negative D1_E* code for rejected arguments.
 * The library allocates no memory; its only global state is the device work buffer
 * that d1_ppo_step_static owns (one per GPU, see there).
 */
#ifndef D1HIP_H
#define D1HIP_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define D1_W 80
#define D1_H 70
#define D1_N 5600
#define D1_VIEW 15                    /* 15x15 window, radius 7 */
#define D1_OBS_CH 8                   /* wall, floor, visible, monster kind+1, monster hp, player hp, stairs, frontier */
#define D1_OBS_BYTES (D1_VIEW * D1_VIEW * D1_OBS_CH)   /* 1800 */
#define D1_ACTIONS 19
#define D1_OUT 8                      /* reward, done, clear, killed, hp, ticks, death, timeout (gpu-d1/src/learn.cu:590-592) */
#define D1_MAX_MONSTERS 64

#define D1_E_ARG (-1)                 /* null pointer, bad size or bad mode */
#define D1_E_CONFIG (-2)              /* config outside the supported ranges */

/* Monster kind: speed, damage, to-hit, shield bypass (gpu-d1/src/sim.h:61-63). */
typedef struct D1Kind { int32_t speed, damage, tohit, bypass; } D1Kind;

/* Runtime rules. The first block is the reference's sim::Config minus its
 * `player` position (gpu-d1/src/sim.h:64-67, packed by gpu-d1/scripts/learn_env.py:67-71);
 * the rest are the task switches that the reference selects with -D flags
 * (gpu-d1/Makefile:14-95, gpu-d1/branches/d1-stairs-v2/scripts/assets.py:5). */
typedef struct D1Config {
    int32_t count;            /* monsters per world, 1..max_monsters of the state layout */
    int32_t hp, ac100, ev100, sh100, shield_limit, regen, repair;
    int32_t gdr[2];           /* floor((65536*(ac+j))^(1/4)) for the two AC roundings */
    D1Kind kinds[6];
    int32_t limit;            /* deadline in physical turns */
    int32_t rng_mode;         /* 0: PCG32 per env (reference stream), 1: Philox4x32-10 counter RNG */
    int32_t level_mode;       /* 0: one shared map from D1Tables, 1: generated level per env */
    int32_t roster_mode;      /* 0: kind i%6 and HP {8,10,12,16,12,10}[i%6]; 1: kind U{0..5}, HP U[hp_lo,hp_hi] */
    int32_t hp_lo, hp_hi;
    int32_t awake_pct;        /* monsters awake at spawn: 0 none, 100 all (no draw), else U{0..99} < pct */
    int32_t wake_los;         /* 1: waking needs the monster's LOS to the player, 0: Chebyshev <= 6 only */
    int32_t stairs;           /* 0 or 3 stairs placed per episode */
    int32_t clear_on_kill_all;/* 1: killing every monster also clears the level */
    int32_t explore_milli, kill_milli, clear_milli, death_milli, step_milli;
    float turn_cost;          /* subtracted per physical turn after the milli sum */
} D1Config;

/* Static tables. `floor`/`cells` are used when level_mode == 0 (byte per cell,
 * row-major, cells = spawnable floor in increasing cell order); `ray_slots` is the
 * [11][64] uint64 per-target LOS ray table (blocker bit j = y*8+x of the +x/+y
 * quadrant), always required. */
typedef struct D1Tables {
    const uint8_t *floor;
    const uint8_t *cells;
    const uint64_t *ray_slots;
    int32_t nslots;           /* 11 for the native ray export */
} D1Tables;

/* Bytes per env of the state row for a given monster capacity (8, 16, 40 or 64). */
int d1_state_bytes(int max_monsters);
int d1_obs_bytes(void);
int d1_action_size(void);
int d1_out_size(void);
int d1_config_bytes(void);

/* Replaces learn_init (gpu-d1/src/learn.cu:649-660): seeds env i's RNG
 * (PCG: seed(mix(seed+i), i+1); counter: key=seed, env=i), builds or copies its
 * level, runs the episode reset and writes the first observation and hash.
 * `state` is uint8 [n, d1_state_bytes(max_monsters)]. */
int d1_init(void *state, int n, int max_monsters, const D1Config *cfg, const D1Tables *tab,
            uint64_t seed, uint8_t *obs, uint32_t *hash, void *stream);

/* Replaces learn_step / learn_step_active (gpu-d1/src/learn.cu:661-670,
 * gpu-d1/branches/d1-stairs-v2/src/learn.cu:853-875): one joint action per env
 * (int64, as the reference's trainer passes them; its low 32 bits are the action as a
 * signed int, as the reference's int parameter takes it, and values outside the action
 * set are invalid actions), then the observation of the post-step (post-reset when done)
 * state. `out` is float [n, D1_OUT].
 * `active` may be null; an inactive env keeps its state and all its output
 * rows untouched and consumes no RNG (gpu-d1/scripts/test_fast_frontier.py:89-100). */
int d1_step(void *state, int n, int max_monsters, const D1Config *cfg, const D1Tables *tab,
            const int64_t *actions, uint8_t *obs, float *out, uint32_t *hash,
            const uint8_t *active, void *stream);

/* Replaces learn_heuristic of the v1 library (gpu-d1/src/learn.cu:599-621,638-640,671-673;
 * gpu-d1/scripts/learn_env.py:114, heuristic()): the v1 pursuit controller's action for
 * each world, written to actions[n] (int64). It attacks the weakest adjacent living monster
 * (lowest HP, then the first direction N, E, S, W, NE, SE, SW, NW), else steps to the first
 * neighbour one floor-BFS layer closer to the nearest living monster (lowest index among
 * the nearest), else waits. joint = 0 writes the v1 action (0-7 direction, 8 wait); joint
 * = 1 writes the joint action d1_step takes for it on the same world (a direction into a
 * living monster's cell is ATTACK 8 + d, another direction MOVE d, 8 is WAIT 16). The
 * state is read only; the reference's gpu = 0 host loop has no counterpart here. */
int d1_heuristic(const void *state, int n, int max_monsters, const D1Config *cfg, int joint,
                 int64_t *actions, void *stream);

/* ---- the reference's monster-wait benchmark workload (gpu-d1/src/bench.cu) ----
 * A stationary player at `player` on one map, `count` (<= 64) awake monsters spawned from
 * starts[fixture*64 + i], the static distance-from-player field `dist` (65535 =
 * unreachable), cfg's player stats and kinds (monster i has kind i%6; task switches are
 * ignored). World rows are d1_wait_bytes() each. */
typedef struct D1WaitMap {
    const uint8_t *floor;     /* byte per cell */
    const uint16_t *dist;     /* distance from `player` per cell */
    const int16_t *starts;    /* [2][64] spawn cells: contact, approach */
    int32_t player;
} D1WaitMap;
int d1_wait_bytes(void);
/* Replaces State::init (gpu-d1/src/bench.cu:151-166): world w seeded with
 * PCG seed(mix(seed+w), w+1); scenario 0 contact, 1 approach, 2 mixed (fixture w%2 and
 * (w*7)%32 warm-up waits). */
int d1_wait_init(void *worlds, int n, int count, const D1Config *cfg, const D1WaitMap *map, uint64_t seed,
                 int scenario, void *stream);
/* `steps` waits per world (sim::step, gpu-d1/src/sim.h:276-295); trace (optional) is
 * uint32 [n, steps] world digests after each wait. */
int d1_wait_run(void *worlds, int n, int count, const D1Config *cfg, const D1WaitMap *map, int steps,
                uint32_t *trace, void *stream);

/* Map compiler's LOS flattening (gpu-d1/scripts/compile_corpus.py:56-93,
 * gpu-d1/scripts/compile_fixture.py:31-48): for each of n_maps byte maps floor[m*5600+p],
 * los[(m*5600 + origin)*10 + w] gets the 17x17 bitset (bit (dy+8)*17+dx+8) of cells seen
 * from `origin` by the ray table in `rays` (ray_slots/nslots; floor/cells unused). This
 * is the `los` table of the learning-task library (include/d1learn.h). */
int d1_los_table(const uint8_t *floor, int n_maps, const D1Tables *rays, uint32_t *los, void *stream);

/* Map compiler's distance rows (gpu-d1/scripts/compile_corpus.py:30-52,
 * gpu-d1/scripts/compile_fixture.py:50-66): for each of the n source cells, BFS over the
 * 8-connected floor cells of floor[5600] (nonzero = floor); dist[i*5600 + p] = the BFS
 * distance of cell p from sources[i], 65535 where unreached (every cell of the row is
 * written; a source outside 0..5599 leaves its row unreached). */
int d1_distance_rows(const uint8_t *floor, const int16_t *sources, int n, uint16_t *dist, void *stream);

/* Categorical sampling with the counter RNG; replaces torch.distributions.Categorical
 * sample/log_prob in the rollout (gpu-d1/scripts/run_ring_ablations.py:350-351).
 * logits: float [n, k] (row stride `ld` floats), 1 <= k <= 64. For env i the uniform
 * is u = (w >> 8) * 2^-24 with w = word 0 of Philox4x32-10(ctr={0, t, i, 3}, key=seed);
 * the action is the first j with u < cumsum_j(softmax(logits)) (fp32, left to right),
 * else k-1. Writes int64 actions and fp32 log-probabilities (either may be null). */
int d1_sample(const float *logits, int n, int k, int ld, uint64_t seed, uint32_t t,
              int64_t *actions, float *logp, void *stream);
/* d1_sample with the counter step read from device memory: t = *t_dev + t_add (same
 * result as d1_sample with that t). A rollout captured in a HIP graph keeps its step
 * counter on the device and advances it on the device, so every replay samples new
 * steps (the reference's loop draws from torch's generator at every call,
 * gpu-d1/scripts/run_ring_ablations.py:350). */
int d1_sample_dev(const float *logits, int n, int k, int ld, uint64_t seed, const uint32_t *t_dev, uint32_t t_add,
                  int64_t *actions, float *logp, void *stream);

/* Autoregressive two-stage sample (the type-then-direction head of
 * gpu-d1/branches/autoregressive-actions-v1/scripts/tactical_models.py:8-30, generalised
 * to nv verbs x nt targets): verb from verb_logits [n, ldv], then target from
 * target_logits [n][nv][nt] (row stride ldt) of that verb; uniforms are Philox words 0/1
 * of ctr={0, t, i, 3}. Writes verb, target, the env action (verb 0/1 + a Chebyshev-1
 * target of the 5x5 grid -> MOVE d / ATTACK 8+d, other targets -1; verb 2/3/4 ->
 * 16/17/18; verbs 5-7 -> 16) and log p(verb) + log p(target | verb). */
int d1_sample_ar(const float *verb_logits, int nv, int ldv, const float *target_logits, int nt, int ldt, int n,
                 uint64_t seed, uint32_t t, int32_t *verb, int32_t *target, int64_t *action, float *logp,
                 void *stream);

/* Rollout policy forward as one MFMA kernel: logits, value = head(relu(relu(obs W1^T + b1)
 * W2^T + b2)) for obs uint8 [M, 1800] (8-byte aligned), hidden 256, a 17-row head (16
 * logits + value); bf16 weights and biases in the torch Linear layout, fp32 accumulation,
 * each layer's output rounded to bf16 (round to nearest even) as the bf16 torch forward
 * rounds it, then logits fp32 [M, 16] (16-byte aligned) and value fp32 [M].
 * Replaces the bf16 rollout forward of the policy (gpu-d1/scripts/run_ring_ablations.py:
 * 209-223 at BASELINE's 1800 -> 256 -> 256 ReLU shape): widening, three GEMMs, dtype copy.
 * The weights are first packed into operand order, once per weight update:
 * d1_policy_pack(w1 [256,1800], w2 [256,256], w3 [17,256], wpk) with wpk holding
 * d1_policy_packed_elems() bf16 values (16-byte aligned). */
int64_t d1_policy_packed_elems(void);
int d1_policy_pack(const void *w1, const void *w2, const void *w3, void *wpk, void *stream);
int d1_policy_fwd(const uint8_t *obs, int M, const void *wpk, const void *b1, const void *b2, const void *b3,
                  float *logits, float *value, void *stream);
/* d1_policy_fwd followed by the counter-RNG sample of every row in the same kernel: the
 * actions and log-probabilities d1_sample / d1_sample_dev would draw from those logits at
 * step t = (t_dev ? *t_dev : 0) + t_add (bit-identical), without the logits round trip
 * through memory (logits may be null). Replaces policy forward + Categorical.sample /
 * log_prob of the rollout loop (gpu-d1/scripts/run_ring_ablations.py:347-351). */
int d1_policy_fwd_sample(const uint8_t *obs, int M, const void *wpk, const void *b1, const void *b2, const void *b3,
                         uint64_t seed, const uint32_t *t_dev, uint32_t t_add, float *logits, float *value,
                         int64_t *actions, float *logp, void *stream);
/* The autoregressive verb x target policy (BASELINE C5; the reference's two-stage head,
 * gpu-d1/branches/autoregressive-actions-v1/scripts/tactical_models.py:8-48, at 8 verbs x 25
 * targets with a 16-wide verb embedding and a 64-unit tanh target MLP) as one kernel: the
 * trunk above, a 17-row head holding the 8 verb logits (rows 0-7, rows 8-15 zero) and the
 * value (row 16), then verb ~ softmax(verb logits) and target ~ softmax(t2 . tanh(t1[:, :256]
 * . h2 + t1 bias + ev[verb]) + t2 bias) with the two-stage counter-RNG draw of d1_sample_ar
 * (bit-identical on the same logits), at step t = (t_dev ? *t_dev : 0) + t_add. Writes
 * action (d1_sample_ar's env action), logp = log p(verb) + log p(target | verb) and value;
 * verb, target, verb_logits [M, 8] (16-byte aligned) and the drawn verb's target_logits
 * [M, 25] when not null. Pack once per weight update with d1_policy_ar_pack(w1, w2, w3 [17,256]
 * (verb rows 0-7, value row 16), t1 [64, 272], t2 [25, 64], ev [8, 64] = t1[:, 256:] .
 * embedding^T (bf16), wpk of d1_policy_ar_packed_elems() bf16); bt = t1 bias [64] then t2
 * bias [25] (bf16, 8-byte aligned). Replaces the policy forward + the two-stage sample of the
 * reference's rollout (tactical_models.py:39-48 and run_ring_ablations.py:347-351 of that
 * branch). */
int64_t d1_policy_ar_packed_elems(void);
int d1_policy_ar_pack(const void *w1, const void *w2, const void *w3, const void *t1w, const void *t2w, const void *ev,
                      void *wpk, void *stream);
int d1_policy_fwd_sample_ar(const uint8_t *obs, int M, const void *wpk, const void *b1, const void *b2, const void *b3,
                            const void *bt, uint64_t seed, const uint32_t *t_dev, uint32_t t_add, float *value,
                            int64_t *action, float *logp, int32_t *verb, int32_t *target, float *verb_logits,
                            float *target_logits, void *stream);

/* D4 camera augmentation of the uint8 observation (the reference's EpisodeSymmetry,
 * gpu-d1/branches/autoregressive-actions-v1/scripts/symmetry.py:10-70, restated for the
 * 15x15x8 window): for env i with group g = groups[i] (0..7; x mirrored when g >= 4, then
 * g%4 quarter turns (x, y) -> (-y, x) about the centre cell, x east, y south), out cell
 * T_g(c) = obs cell c (all 8 channels). obs and out are distinct, 8-byte aligned. */
int d1_obs_d4(const uint8_t *obs, const int32_t *groups, int n, uint8_t *out, void *stream);

/* Widen `count` uint8 observation bytes to bf16 (exact), for the policy trunk.
 * count must be a multiple of 16 and both pointers 16-byte aligned. */
int d1_obs_to_bf16(const uint8_t *obs, void *out_bf16, int64_t count, void *stream);

/* One PPO minibatch update of the 1800 -> 256 -> 256 ReLU policy with a 17-wide head
 * (16 logits + value): gather through the sample order, forward, clipped-surrogate +
 * value + entropy loss, backward, global-norm clipping and Adam on fp32 masters
 * (gpu-d1/scripts/train_clear.py:160-172, gpu-d1/scripts/run_ring_ablations.py:363-372),
 * computed as torch bf16 autocast does: bf16 operands, fp32 accumulation, bf16 results.
 *
 * Minibatch i = cursor[0] covers samples perm[i*mb .. i*mb+mb) of the rollout buffer; each
 * call advances cursor[0] on the device, so a captured graph of several calls walks
 * consecutive minibatches. A call whose minibatch would end past n changes nothing.
 * Graph-safe: no memsets, no atomic read-modify-writes; every reduction has a fixed order
 * (bit-reproducible).
 *
 * Parameters live in flat buffers (element offsets off_* into p / pb / g / m / v, each a
 * multiple of 8): l1.weight [256,1800], l1.bias [256], l2.weight [256,256], l2.bias [256],
 * head.weight [17,256], head.bias [17] (torch Linear layouts). `work` holds, besides
 * scratch, copies of the bf16 weights in the order the kernels read them: d1_ppo_prepare
 * writes them from pb (once before the first step, and again whenever the parameters are
 * changed outside d1_ppo_step); every step refreshes them with its updated weights. */
typedef struct {
    const uint8_t *obs;             /* [n, 1800] uint8 observations (8-byte aligned) */
    const int64_t *perm;            /* [n] sample order, entries in [0, n) */
    int32_t *cursor;                /* [2] device ints: cursor[0] = minibatch number, cursor[1] = scratch */
    const int64_t *actions;         /* [n] */
    const float *logp_old, *adv, *ret;   /* [n] */
    int64_t n;                      /* samples in the buffer, < 2^31 */
    int32_t mb;                     /* minibatch size, a multiple of 1024 */
    int32_t pad0;
    float *p;                       /* fp32 master parameters (16-byte aligned, like every flat buffer) */
    void *pb;                       /* bf16 copy */
    void *g;                        /* bf16 gradients written by the call */
    float *m, *v;                   /* Adam moments */
    int64_t nparams;                /* a multiple of 4 */
    int64_t off_w1, off_b1, off_w2, off_b2, off_w3, off_b3;
    float *step;                    /* [3]: [0] Adam step count (torch.optim.Adam semantics, no decay), [1] scratch,
                                       [2] steps skipped since the first non-finite loss or gradient norm (sticky:
                                       while non-zero every step is skipped; the caller clears it) */
    float *loss_parts;              /* [mb/32 * 4]: per 32 samples the sums of pg, 0.5*(v-R)^2, entropy */
    void *work;                     /* d1_ppo_work_bytes(mb) bytes of device memory, 256-byte aligned */
    int64_t work_bytes;
    float clip, vcoef, ecoef, max_grad_norm, lr, beta1, beta2, eps;
    float *z_out;                   /* optional [mb, 17]: the head outputs the loss was computed from (16 logits
                                       and the value, each the bf16-rounded head output widened to fp32), in
                                       minibatch order; null to skip */
} D1PPOStep;
int64_t d1_ppo_work_bytes(int mb);
int d1_ppo_prepare(const D1PPOStep *s, void *stream);
int d1_ppo_step(const D1PPOStep *s, void *stream);

/* No counterpart in the reference. For callers that cannot allocate device memory (code
 * under graph capture, tight serving loops, harnesses that forbid hipMalloc): d1_ppo_step
 * with the work buffer owned by the library, so s->work and s->work_bytes are ignored.
 * The buffer is one file-scope device array per GPU of d1_ppo_work_bytes(D1_PPO_STATIC_MAX_MB)
 * bytes (51,710,464), held from the library's load until the process ends; a larger s->mb
 * returns D1_E_SCRATCH. Each call first rebuilds the packed
 * weight copies from s->pb (as d1_ppo_prepare does) and then runs d1_ppo_step's kernels, so
 * one call equals d1_ppo_prepare + d1_ppo_step on a private work buffer, bit for bit.
 * Every call on one GPU shares that GPU's array: calls that overlap in time on one GPU
 * (two streams, two threads) race and give undefined results; calls in stream order do not.
 * The call itself allocates nothing (no hipMalloc, no library allocation). Its first call on
 * a device resolves that device's array address (hipGetSymbolAddress), which is not a stream
 * operation: make that first call outside stream capture; later calls may be captured. */
#define D1_PPO_STATIC_MAX_MB 8192
#define D1_E_SCRATCH (-4)             /* request larger than the library-owned buffer */
int d1_ppo_step_static(const D1PPOStep *s, void *stream);

/* Reverse-time GAE over a [T, n] rollout (gpu-d1/scripts/run_ring_ablations.py:354-360):
 *   live = 1 - done[t]; delta = reward[t] + (gamma*next)*live - value[t];
 *   gae = delta + (gamma_lambda*live)*gae; adv[t] = gae; next = value[t]
 * with next = bootstrap for t = T-1 and every product rounded separately (fp32).
 * `done` is uint8 [T, n]; returns[t] = adv[t] + value[t]. */
int d1_gae(const float *reward, const uint8_t *done, const float *value, const float *bootstrap,
           int T, int n, float gamma, float gamma_lambda, float *adv, float *returns, void *stream);

#ifdef __cplusplus
}
#endif
#endif
