/*
 * qqt_hip.h - C ABI of the MI355X rollout hot path (libqqt_hip.so).
 *
 * Every entry point takes plain device pointers and sizes plus a hipStream_t
 * (passed as void*), launches asynchronously on that stream, never allocates
 * and never synchronises.  It returns 0 on success or a negative QQT_E* code;
 * qqt_last_error() then describes the failure (thread-local).
 *
 * Device state of one batched sim (N envs, H x W grid, P players), all
 * env-major:
 *   cells   int32 [N][H*W]  cell word: bits 0-7 fuse (0..255), 8-15 owner
 *                           (int8, -1 = none), 16-23 bomb_blast, 24 wall,
 *                           25 brick, 26 crate, 27 recycle-crate
 *   players int32 [N][P][16] player record (slots QQT_P_*; float slots hold
 *                           IEEE-754 bits)
 *   envs    int32 [N][4]    t, crate_prob (float bits), map_kind, reserved
 * Reference layout (N,H,W) / (N,P) tensors are converted by the Python host
 * layer (qqtsim/state.py).
 */
#ifndef QQT_HIP_H
#define QQT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QQT_ABI_VERSION 25

#define QQT_OK 0
#define QQT_E_ARG (-1)      /* bad argument (shape, null pointer, range) */
#define QQT_E_LAUNCH (-2)   /* kernel launch failed */
#define QQT_E_UNSUPPORTED (-3) /* grid/player combination not compiled */

/* player record slots */
enum {
  QQT_P_Y = 0, QQT_P_X = 1, QQT_P_ALIVE = 2, QQT_P_HP = 3, QQT_P_SINCE_BOMB = 4,
  QQT_P_BOMBS_CAP = 5, QQT_P_BLAST_CAP = 6, QQT_P_SPD = 7, QQT_P_INVULN = 8,
  QQT_P_COMBO = 9, QQT_P_LAST_HIT = 10, QQT_P_PENDING_LOST = 11,
  QQT_P_LO_BOMBS = 12, QQT_P_LO_BLAST = 13, QQT_P_LO_SPD = 14, QQT_P_SLOTS = 16
};
/* env record slots */
enum { QQT_E_T = 0, QQT_E_CRATE_PROB = 1, QQT_E_MAP_KIND = 2, QQT_E_SLOTS = 4 };

/* Rule constants of one sim; mirrors the SimConfig fields the tick reads
 * (reference sim/config.py:102-443).  Float fields are the float32 values
 * the reference's tensor ops use (Python doubles rounded once). */
typedef struct qqt_sim_config {
  int32_t height, width, n_players;
  int32_t fuse, blast, max_steps, max_chain, chain_cap_rounds;
  int32_t max_hp, invuln_ticks, hit_attr_penalty, place_dist_cooldown;
  int32_t growth_bombs_max, growth_blast_max, corridor, timeout_draw, win_hp_scaled;
  float radius, step_len, pos_hi_y, pos_hi_x;
  float step_penalty, hit_reward, win_bonus, win_per_hp, danger_penalty, brick_reward;
  float place_cover_reward, place_chain_reward, place_dist_reward, place_dist_radius;
  float chain_time_factor, chain_time_rest;   /* rest = 1 - chain_time_factor */
  float combo_reward, combo_gap_factor;
  float growth_speed_step, growth_speed_max, hit_speed_drop; /* drop = pen*step */
  float recycle_crate_prob, growth_crate_prob;
  /* reset template (qqtsim/maps.py MapSpec) */
  int32_t map_kind, swap_spawns, bombs_lo, bombs_hi, blast_lo, blast_hi, spawn_cooldown;
  float brick_p, spawn_speed;
  /* the reference's map modes (map_kind QQT_MAP_REFERENCE; BatchedSim.reset_,
   * sim/torch_sim.py:178-420, and sim/mapgen.py:15-242) */
  int32_t top_wall_rows, random_wall_rows, corridor_width, open_obstacle_max;
  int32_t ring_center_h, ring_center_w, open_crate_cross, max_bombs;
  int32_t growth_bombs_start, growth_blast_start, open_growth_bombs, open_growth_blast;
  int32_t opp_growth_bombs, opp_growth_blast;
  float thr_pure, thr_open, thr_ring;   /* map-type thresholds: float32 of the cumulative
                                           fractions pure, +open, +ring (corridor mode) */
  float wall_density, ring_brick_density, ring_crate_prob;
  float growth_speed_start, open_growth_speed, opp_growth_speed, opp_hist_mult;
  /* spawns of the corridor, open and ring layouts (SimConfig.spawn_pos /
   * ring_spawns, float32) and their cells r*W + c (taken from the double
   * values, like cfg.spawn_cells()) */
  float ref_spawn_y[3][4], ref_spawn_x[3][4];
  int32_t ref_spawn_cell[3][4];
} qqt_sim_config;

/* map_kind values */
#define QQT_MAP_PILLARS 0    /* template: border + even/even pillars, bricks w.p. brick_p */
#define QQT_MAP_OPEN 1       /* template: empty grid */
#define QQT_MAP_REFERENCE 2  /* the reference's corridor / open / ring modes */

/* modes of qqt_tick */
#define QQT_MODE_STEP 0     /* one tick, then auto-reset, observe and masks */
#define QQT_MODE_OBSERVE 1  /* observe + masks of the current state only */
#define QQT_MODE_RESET 2    /* map reset (map_kind) where reset_mask, then observe */
#define QQT_MODE_PROBE 3    /* largest bomb_blast after this tick's placement */
#define QQT_MODE_FLUSH 4    /* recycle flush (each player's pending lost growth becomes
                               recycle crates on random free cells), then observe */

typedef struct qqt_tick_args {
  int32_t n_envs;
  int32_t mode;
  int32_t auto_reset;         /* STEP: reset envs that finish */
  int32_t resolve_tiers;      /* blast tiers the explosion resolves (see sim.py) */
  float explore_coef;         /* annealing alpha of the shaping rewards */
  float danger_coef;          /* explore_coef * danger_penalty (rounded once) */
  uint64_t seed;              /* Philox key */
  uint32_t tick;              /* keys per-tick uniforms (crates) */
  uint32_t epoch;             /* keys template draws of this call's resets
                                 (FLUSH: the flush counter keying the cell draws) */
  /* state (in/out) */
  int32_t* cells;
  int32_t* players;
  int32_t* envs;
  /* inputs */
  const int64_t* actions;     /* STEP: [N][P][2] move, bomb (int64) */
  const int8_t* actions_i8;   /* or the same as int8 (one of the two) */
  const float* crate_u;       /* STEP: [P][2][N] or NULL = Philox stream */
  const uint8_t* reset_mask;  /* RESET: [N] */
  /* outputs (NULL = not wanted, except obs/masks in STEP/OBSERVE/RESET) */
  float* reward;              /* [N][P] */
  uint8_t* done;              /* [N] */
  int32_t* n_alive;           /* [N] */
  uint8_t* died;              /* [N][P] */
  uint8_t* winner;            /* [N][P] */
  uint32_t* covered;          /* [N][8] bitset of the tick's flame cover */
  uint32_t* triggered;        /* [N][8] bitset of the tick's exploded bombs */
  uint16_t* obs;              /* [N][5P+4][H][W] float16 bits */
  uint8_t* move_mask;         /* [N][P][5] */
  uint8_t* bomb_mask;         /* [N][P][2] */
  int32_t* probe_out;         /* PROBE: [N] largest bomb_blast */
  uint8_t* damaged;           /* STEP: [N][P] 1 if the player's hp fell this tick,
                                 judged after the auto-reset like the collect
                                 loop's (hp0 - sim.hp).clamp(min=0) > 0
                                 (train/ppo.py:251); or NULL */
  const uint8_t* recycle_excl; /* FLUSH: [H*W] 1 = never a recycle crate (spawn
                                 neighbourhoods, the open-mode cross band) */
  int32_t opp_boost;          /* QQT_MAP_REFERENCE resets: player 1's start tier
                                 (0 as player 0, 1 x opp_hist_mult, 2 opp_growth_*;
                                 BatchedSim.set_opp_boost, sim/torch_sim.py:422-453) */
  float* danger_out;          /* OBSERVE: [N][H][W] float32 danger map of the current
                                 state (blast.danger_map as BatchedSim._danger_c
                                 computes it, sim/torch_sim.py:732-762), or NULL */
  int32_t* tick_stats;        /* STEP: [N][4], 16-byte aligned, or NULL: slots 0-2 of env
                                 n are incremented by this launch's exploded bombs
                                 (info["trig"] cells), deaths (info["died"]) and
                                 auto-reset (1 if the env was done and reset) of env n;
                                 slot 3 is left as it is.  For benchmark harnesses that
                                 report what their timed ticks did (sum over envs after
                                 the launches); no reference counterpart. */
  int8_t* reach_caps;         /* STEP: int8 [N rounded up to a multiple of 16], zeroed
                                 once by the caller, or NULL: maxima of the blast cap
                                 of player reach_pid after the tick and its auto-reset,
                                 one per group of E consecutive envs (E = 2 up to 8192
                                 envs, else 4), in the first ceil(N / E) entries (the
                                 rest is left as it is).  The astar bot's next call
                                 reduces them to the batch max (qqt_bot_args
                                 reach_mode 3) instead of a reduction launch of its own. */
  int32_t reach_pid;
} qqt_tick_args;

/* MLP actor/critic forward (+ masked sampling).  Weights are the packed
 * device buffers built by qqtsim/policy.py from an ActorCritic "mlp"
 * state_dict (train/model.py:121-165): fragment-ordered float16 matrices
 * w0 (both players' view-permuted first layers), w1, wh (the three head
 * hidden layers stacked), wf (the three output layers, block diagonal, 16
 * padded rows), the float16 residuals of w1/wh/wf (the later layers run as
 * hi/lo pairs), and float32 vectors.  w0 is [tile][64-deep K block][lane][16],
 * zero at K >= k0 (the act kernel's K blocks read past k0 from inside the
 * row and rely on those zero weights); w1/wh/wf are [tile][32-deep K step][lane][8] in the K order in which one
 * layer's MFMA output tiles feed the next (csrc/mlp.hip documents both).
 * Outputs are indexed [row][player slot]. */
typedef struct qqt_mlp_args {
  int32_t batch;             /* rows B */
  int32_t npid;              /* 1: player pid0 only; 2: both players */
  int32_t pid0;
  int32_t sample;            /* 1: draw actions (needs masks) */
  int32_t k0, kblocks0;      /* first-layer width (C*H*W) and ceil(k0/64) */
  int32_t obs_stride;        /* elements between observation rows (even) */
  int32_t mm_row_stride, mm_pid_stride;  /* move mask [row*rs + pid*ps + k] */
  int32_t bm_row_stride, bm_pid_stride;  /* bomb mask */
  uint64_t seed;             /* Philox key of the policy uniforms */
  uint32_t tick;             /* counter word of the policy uniforms */
  int32_t w0_players;        /* players whose first layers w0 holds (pid0, npid < it) */
  const uint16_t* obs;       /* [B][obs_stride] float16 bits, 4-byte aligned */
  const uint16_t *w0, *w1, *wh, *wf;       /* float16 (hi) fragments */
  const uint16_t *w1_lo, *wh_lo, *wf_lo;   /* float16 residuals w - hi */
  const float *b0, *ln1_w, *ln1_b, *b1, *ln2_w, *ln2_b, *bh, *bf;
  const uint8_t* move_mask;
  const uint8_t* bomb_mask;
  const float* uniforms;     /* [B][out_slots][2] (move, bomb) or NULL = Philox */
  int64_t* actions;          /* [B][out_slots][2] or NULL */
  int8_t* actions_i8;        /* [B][out_slots][2] or NULL */
  float* logp_out;           /* [B][out_slots] or NULL */
  float* value_out;          /* [B][out_slots] or NULL */
  float* logits_out;         /* [B][out_slots][8]: 5 move, 2 bomb, value; or NULL */
  int32_t out_slots;         /* player slots per output row (0 = npid) */
  int32_t out_slot;          /* slot written when npid == 1 */
  float* z1_out;             /* [B][128] or NULL.  When set (npid 1, sample 0) the
                                launch computes the first layer only,
                                z1 = obs W0[pid]^T + b0 in float32 (the training
                                forward's input to LayerNorm 1), and writes
                                nothing else */
  const int64_t* row_index;  /* [B] or NULL: row b of the batch is observation row
                                row_index[b] (a PPO minibatch read in place from the
                                flattened rollout buffer, train/ppo.py:406-408,
                                without a gather); entries are clamped into
                                [0, obs_rows), so no index reads outside obs */
  int64_t obs_rows;          /* rows of obs (> 0 when row_index is set) */
  /* Sparse first layer.  When `sparse` is 1 and the shapes qualify (no
     z1_out; sampling, or fewer than 65,536 rows; npid 1 or 2; 128 <= cells
     <= 192; channels <= 16 with k0 = channels * cells; at most two dense
     channels), the launch computes z1 = W0 x + b0 per workgroup of 22 rows
     and both players as
       the sum over the dense channels c of W0[:, c] x[c] on MFMA (the
       float16 hi and lo parts of the weights times the exact float16
       observation), plus
       the sum over the nonzero cells k of every other channel of
       x[k] * W0[:, column of k in the player's view] (float16 columns,
       float32 sums).
     Otherwise (or when a workgroup's rows hold more nonzero cells than its
     lists take) the first layer is the dense product.  Both give the same
     function up to float rounding. */
  int32_t sparse;
  int32_t channels, cells;   /* C and H*W (k0 = channels * cells) */
  uint32_t dense_mask;       /* storage channels multiplied on MFMA (<= 2 bits) */
  const uint16_t* w0g;       /* [k0][128] float16: row k = W0[:, k] in the network's
                                own (view) input order */
  const uint16_t* w0d;       /* [C][8 tiles][ceil(cells/32)][2 planes][64 lanes][8]
                                float16 MFMA A fragments of view channel j: lane
                                (r = lane%16, g = lane/16) holds W0[16 tile + r]
                                [j*cells + 32 s + 8 g + i] (0 past the channel),
                                plane 0 float16(w), plane 1 float16(w - plane 0) */
  int8_t vmap[4][16];        /* view channel of storage channel c for player p
                                (the inverse of the view permutation) */
} qqt_mlp_args;

/* astar rule bot for one player (sim/bots.py:267-508, astar_attack with no
 * behaviour modes and no crate eating).  Reads the sim state, the tick's
 * float16 observation (danger channel 2P+1) and the player's legality masks;
 * writes slot `pid` of the (N, P, 2) action buffer. */
typedef struct qqt_bot_args {
  int32_t n_envs;
  int32_t pid;                /* the bot's player id */
  uint64_t seed;              /* Philox key of the noise uniforms */
  uint32_t tick;              /* counter word of the noise uniforms */
  int32_t reach_mode;         /* chain-check reach: 0 = the bot's own blast cap;
                                 1 = the batch max of the bot's blast cap (the
                                 reference's rule), computed by this call into
                                 reach[reach_slot & 1]; 2 = the value already in
                                 reach[0]; 3 = that batch max from the caps a STEP
                                 tick wrote to reach_caps (its reach_pid = pid, the
                                 padding 0), when nothing changed the state since
                                 that tick */
  int32_t reach_slot;         /* mode 1: reach is int32[2], both INT32_MIN before
                                 the first call; call k passes slot k (any
                                 counter that alternates): the call max-reduces
                                 into reach[slot & 1] and resets the other slot
                                 to INT32_MIN for the next call */
  const int32_t* cells;       /* sim state, layout above */
  const int32_t* players;
  const uint16_t* obs;        /* [N][5P+4][H][W] float16 bits */
  const uint8_t* move_mask;   /* [N][P][5] */
  const uint8_t* bomb_mask;   /* [N][P][2] */
  const float* uniforms;      /* [N][5] noise uniforms, or NULL = Philox stream 7 */
  int32_t* reach;             /* device int32[2] (mode 1) or scalar (mode 2) */
  const int8_t* reach_caps;   /* mode 3: the tick's cap maxima, int8 [N rounded up to
                                 16], 16-byte aligned, zero past the tick's entries */
  int64_t* actions;           /* [N][P][2], slot pid written; or NULL */
  int8_t* actions_i8;         /* same as int8; or NULL */
  int8_t* mode;               /* [N] behaviour mode per env, 0 approach / 1 flee
                                 (sim/bots.py:433-443, 496-503), or NULL = always
                                 approach (make_bot(..., mode=False)) */
  int32_t* mode_timer;        /* [N] countdown of the mode ticker (sim/bots.py:241-264) */
  uint32_t mode_tick;         /* this call's ticker count (1, 2, ...): every timer
                                 counts down by one and, on multiples of 16, envs at
                                 or below 0 draw a new mode (probability 1/2 each)
                                 and timer (60 .. 239) from Philox stream 9 (counter
                                 env, mode_tick); 0 = modes as given, no ticker step */
  int32_t reserved;
} qqt_bot_args;

/* ABI version (QQT_ABI_VERSION). */
int qqt_abi_version(void);

/* Last error message of this thread ("" if none). */
const char* qqt_last_error(void);

/* One launch of the fused tick kernel.  Replaces, on the device, the
 * reference's BatchedSim.step (sim/torch_sim.py:895-1261) followed by
 * BatchedSim.observe (:605-627) and BatchedSim.legal_mask (:636-645), plus
 * reset_ (:178-420) with template maps, per `mode`. */
int qqt_tick(const qqt_sim_config* cfg, const qqt_tick_args* args, void* stream);

/* One launch of the MLP forward with optional masked sampling.  Replaces
 * ActorCritic.act (train/model.py:230-245) for one or both players (obs is
 * shared, so both players' first layers are one GEMM), ActorCritic.forward
 * (:167-196) when sample = 0. */
int qqt_mlp_act(const qqt_mlp_args* args, void* stream);

/* One launch of the astar bot for player args->pid.  Replaces
 * astar_attack(sim, obs, mmask, bmask, pid) (sim/bots.py:267-508) with its
 * two _dijkstra_field cost fields (:179-238); the 0.05 * torch.rand(n, 5)
 * noise (:355) comes from `uniforms` or the Philox stream. */
int qqt_bot_act(const qqt_sim_config* cfg, const qqt_bot_args* args, void* stream);

/* Generalised advantage estimation over a filled rollout buffer: the
 * reverse-time scan of compute_gae (train/ppo.py:101-110) in the reference's
 * float32 operation order, one thread per env:
 *   delta = (rew[t] + (gamma * next_val) * nt) - val[t],  nt = 1 - done[t]
 *   gae   = delta + (gamma_lam * nt) * gae;  adv[t] = gae;  ret[t] = gae + val[t]
 * with next_val = last_val at t = steps - 1, val[t + 1] before. */
typedef struct qqt_gae_args {
  int32_t steps;              /* T */
  int32_t n_envs;             /* N */
  float gamma;                /* float32(gamma) */
  float gamma_lam;            /* float32 rounding of gamma * lam taken in double
                                 (the reference's Python expression) */
  int64_t step_stride;        /* elements between steps of rew and val */
  int64_t env_stride;         /* elements between envs of rew and val */
  const float* rew;           /* e.g. player 0 of a [T][N][P] reward slab */
  const float* val;
  const uint8_t* done;        /* [T][N], 0 or 1 */
  const float* last_val;      /* [N] */
  float* adv;                 /* [T][N] */
  float* ret;                 /* [T][N] */
} qqt_gae_args;

/* One launch of the GAE scan (replaces compute_gae, train/ppo.py:101-110). */
int qqt_gae(const qqt_gae_args* args, void* stream);

/* First-layer weight gradient of the PPO update's backward pass (the
 * product loss.backward() forms for shared.0.weight, train/ppo.py:364-437
 * through train/model.py:121-147), for the view-permuted first layer of
 * one player:  dw0[h][k] = sum_b dz1[b][h] * obs[b][k]  (h < 128, k < k0).
 * float16 MFMA with float32 accumulation; dz1 is multiplied by *dz_scale
 * (a power of two chosen by the caller so that max|dz1| * scale <= 2^14;
 * NULL = 1) before its float16 hi/lo split and the result is divided by it.
 * Deterministic: fixed batch chunks summed in chunk order.  The caller
 * provides the workspace (qqt_l1_grad_workspace_floats floats). */
typedef struct qqt_l1_grad_args {
  int32_t batch;              /* rows B */
  int32_t k0;                 /* observation width C*H*W (even) */
  int32_t obs_stride;         /* elements between observation rows (even) */
  int32_t reserved;
  int64_t workspace_floats;   /* size of workspace */
  const uint16_t* obs;        /* [B][obs_stride] float16 bits, 4-byte aligned */
  const float* dz1;           /* [B][128], 8-byte aligned */
  const float* dz_scale;      /* [1] device float, or NULL */
  float* workspace;
  float* dw0;                 /* [128][k0] */
  const int64_t* row_index;   /* [B] or NULL: row b is observation row row_index[b]
                                 (as in qqt_mlp_args; clamped into [0, obs_rows)) */
  int64_t obs_rows;           /* rows of obs (> 0 when row_index is set) */
} qqt_l1_grad_args;
int64_t qqt_l1_grad_workspace_floats(int32_t batch, int32_t k0);
int qqt_l1_grad(const qqt_l1_grad_args* args, void* stream);

/* qqt_l1_grad without a caller workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  The chunk partials
 * go to a file-scope device array of 64 x 128 x QQT_L1_GRAD_NOALLOC_MAX_K0
 * floats (80 MiB, one per GPU, held until the process ends); `workspace`
 * and `workspace_floats` are ignored.  Any batch size; k0 at most
 * QQT_L1_GRAD_NOALLOC_MAX_K0 (larger is QQT_E_ARG).  The result equals
 * qqt_l1_grad's bit for bit (same plan, same kernels).  The call allocates
 * nothing: its first call on a device looks up the array's address there.
 * Every element of the array that a call reads, the same call wrote first;
 * calls that overlap on one GPU (different streams) race on the array. */
#define QQT_L1_GRAD_NOALLOC_MAX_K0 2560
int qqt_l1_grad_noalloc(const qqt_l1_grad_args* args, void* stream);

/* The PPO minibatch loss and its backward above the first layer, fused
 * (train/ppo.py:401-421 through train/model.py:140-153, 192-196, 215-256):
 * from z1 = x W0^T + b0 per row, LayerNorm/ReLU, Linear(128,128),
 * LayerNorm/ReLU, the three heads, the masked log-probs and entropies, the
 * clipped policy loss, the clipped value loss and the entropy bonus, back to
 * dz1.  float32.  Row outputs feed the weight gradients the caller forms
 * over the minibatch (dW1 = dz2^T h1, dWh = dhy^T h2, output layers from dl
 * and hy, dW0 via qqt_l1_grad on dz1); per 16-row block sums of the
 * LayerNorm parameter gradients and of the loss statistics. */
typedef struct qqt_ppo_args {
  int32_t batch;              /* rows B of the minibatch (the means' divisor) */
  float clip_eps;             /* float32(clip_eps): value clip and clip fraction */
  float ratio_lo, ratio_hi;   /* float32(1 - clip_eps), float32(1 + clip_eps) */
  float value_coef, entropy_coef;
  const float* z1;            /* [B][128] */
  const float *ln1_w, *ln1_b; /* [128] */
  const float *w1, *w1t;      /* shared.3.weight W1 [128 out][128 in] as k-major matrices
                                 [K][N] for the products dh1 = dz2 W1 (K = out) and
                                 z2 = h1 W1^T (K = in), each in MFMA fragments: value i
                                 of lane l in 16-k group g of column tile t is
                                 M[16 g + 4 (l / 16) + i][16 t + l % 16] */
  const float* b1;
  const float *ln2_w, *ln2_b;
  const float *wh, *wht;      /* the heads' hidden layers stacked, Wh [192][128], likewise:
                                 wh for dh2 = dhy Wh (K = 192), wht for hy = h2 Wh^T */
  const float* bh;            /* [192] */
  const float* wf;            /* [8][64]: move rows 0-4, bomb 5-6, critic 7 (each head's
                                 output layer over its own 64 hidden units) */
  const float* bf;            /* [8] */
  const int64_t* actions;     /* [B][2] */
  const uint8_t* move_mask;   /* [B][5] */
  const uint8_t* bomb_mask;   /* [B][2] */
  const float *old_logp, *adv, *ret, *old_val;   /* [B]; adv normalised by the caller */
  float* dz1;                 /* [B][128] */
  float *h1, *dz2, *h2;       /* [B][128] */
  float *hy, *dhy;            /* [B][192] */
  float* dl;                  /* [B][8]: d loss / d (5 move logits, 2 bomb logits, value) */
  float* ln_part;             /* [ceil(B/16)][4][128]: dgamma1, dbeta1, dgamma2, dbeta2 */
  float* stats_part;          /* [ceil(B/16)][5]: sums of -min(surrogates), 0.5 max(value
                                 errors), entropy, old_logp - logp, clipped indicator */
  float* bias_part;           /* [ceil(B/16)][456] or NULL: column sums of dz1 (128), dz2
                                 (128), dhy (192), dl (8) over each 16-row block */
  float* dz1_absmax_part;     /* [ceil(B/16)][128] or NULL: max |dz1| per column and block */
  int32_t t_chunk;            /* 0: dz2, dhy, dl row-major.  A multiple of 16: written
                                 chunk-transposed, element (row r, column c) of an
                                 n-column output at ((r / t_chunk) n + c) t_chunk +
                                 r % t_chunk (each chunk [n][t_chunk], ready for batched
                                 products over the rows; the caller sizes the buffers to
                                 whole chunks and zeroes the last chunk's tail) */
  int32_t reserved;
  const int64_t* row_index;   /* [B] or NULL: the per-row inputs actions, move_mask,
                                 bomb_mask, old_logp, adv, ret and old_val of minibatch
                                 row b are their row row_index[b] (the flattened rollout
                                 buffer's fields, read in place), clamped into
                                 [0, src_rows); z1 and every output stay in minibatch
                                 order */
  int64_t src_rows;           /* rows of those inputs (> 0 when row_index is set) */
} qqt_ppo_args;
int qqt_ppo_grad(const qqt_ppo_args* args, void* stream);

/* Row gather for the PPO update's minibatches (train/ppo.py:406-408,
 * buf.obs[mb] with the flattened buffer): destination row r = source row
 * index[r], row_words 4-byte words each.  Rows whose index lies outside
 * [0, src_rows) are left untouched. */
typedef struct qqt_gather_args {
  int32_t n;                  /* destination rows */
  int32_t row_words;          /* 4-byte words per row */
  int64_t src_rows;           /* rows in src */
  int64_t src_stride, dst_stride;   /* words between rows */
  const uint32_t* src;
  uint32_t* dst;
  const int64_t* index;       /* [n] */
} qqt_gather_args;
int qqt_gather_rows(const qqt_gather_args* args, void* stream);

/* Forward of the cnn actor/critic (train/model.py:79-96, 186-190) with
 * optional masked factored sampling.  Replaces ActorCritic.act / forward for
 * arch "cnn" (:167-196, 230-245) as qqt_mlp_act does for the MLP: the same
 * masks, uniforms and output layout.  Every LayerNorm normalises one sample
 * over all of its values (eps 1e-5) with an elementwise affine of that shape.
 * Weights come in the kernel's operand order.  The 3x3 conv weights are
 * float16 hi / lo planes (w = hi + lo), index [tile][step][lane][8]: lane l
 * holds output 16 tile + l % 16 and 8 consecutive input channels at one
 * tap, the block of lane group g = l / 16: for 16 input channels (conv0
 * padded from 14 with zero weights, and conv 16->32) combination
 * c = 4 step + g, tap c / 2 (taps 3 dy + dx; combinations 18, 19 are zero),
 * channels 8 (c % 2)..; for 32 input channels tap = step, channels 8 g...
 * The 1x1 conv is float16 hi / lo per block of 16 input channels (see
 * c3w).  Linear(1352,128) comes as float16 hi / lo
 * planes [tile][43 steps][lane][8]: lane l holds output 16 tile + l % 16 and
 * inputs 32 step + 8 (l / 16) .. + 7 of the flattened [8][13][13] (inputs
 * 1352..1375 zero).  The other Linear weights are float32
 * [tile][step][lane], lane l holding output 16 tile + l % 16, input
 * 4 step + l / 16.  The 3x3 convs' LayerNorm tables are packed [tile][13
 * rows][lane][4] (value q of lane l in row y: channel 16 tile + 4 (l / 16) +
 * q at position (y, x = l % 16); zero for x >= 13 or past the channel
 * count), 16-byte aligned; the 1x1 conv's are plain [8][13][13].  Two launches on `stream`: the trunk writes each item's
 * flattened features as float16 hi / lo rows into the workspace, the head
 * reads them; calls that overlap on one workspace race. */
#define QQT_CNN_WS_BYTES_PER_ITEM 5504   /* workspace bytes per (row, player) item */
typedef struct qqt_cnn_args {
  int32_t batch;              /* rows B */
  int32_t npid;               /* 1: player pid0 only; 2: both players */
  int32_t pid0;
  int32_t sample;             /* 1: draw actions (needs masks) */
  int32_t obs_stride;         /* elements between observation rows (>= 14*169) */
  int32_t mm_row_stride, mm_pid_stride;  /* move mask [row*rs + pid*ps + k] */
  int32_t bm_row_stride, bm_pid_stride;  /* bomb mask */
  int32_t w_players;          /* player views view_perm holds (pid0, npid < it) */
  uint64_t seed;              /* Philox key of the policy uniforms */
  uint32_t tick;              /* counter word of the policy uniforms */
  int32_t out_slots;          /* player slots per output row (0 = npid) */
  int32_t out_slot;           /* slot written when npid == 1 */
  int32_t reserved;
  const uint16_t* obs;        /* [B][obs_stride] float16 bits, [14][13][13] per row */
  const int32_t* view_perm;   /* [w_players][14]: conv0 input channel j of player p is
                                 observation channel view_perm[p][j] (the reference's
                                 conv0.weight[:, argsort(view_perm)] on the stored obs) */
  const uint16_t *c0w, *c0w_lo;           /* conv0 [1][5][64][8] */
  const float *c0b, *ln0w, *ln0b;         /* [16]; LN [1][13][64][4] */
  const uint16_t *c1w, *c1w_lo;           /* conv 16->32 [2][5][64][8] */
  const float *c1b, *ln1w, *ln1b;         /* [32]; LN [2][13][64][4] */
  const uint16_t *c2w, *c2w_lo;           /* conv 32->64 [4][9][64][8] */
  const float *c2b, *ln2w, *ln2b;         /* [64]; LN [4][13][64][4] */
  const uint16_t *c3w, *c3w_lo;           /* 1x1 64->8 [4 input blocks][64][4]: value j of lane
                                             l is W[l % 16][16 b + 4 (l / 16) + j] (rows 8..15
                                             zero) */
  const float *c3b, *ln3w, *ln3b;         /* [16] (8..15 zero); LN plain [8][13][13] */
  const uint16_t *s0h, *s0l;  /* Linear(1352,128) float16 hi / lo [8][43][64][8] (input
                                 index c * 169 + p of the flattened [8][13][13]) */
  const float* s0b;           /* [128] */
  const float *s1w, *s1b;     /* LayerNorm(128) */
  const float *s3p, *s3b;     /* Linear(128,128) packed [8][32][64]; [128] */
  const float *s4w, *s4b;     /* LayerNorm(128) */
  const float *hp, *hb;       /* heads' hidden layers (move | bomb | critic, 192 outputs)
                                 packed [12][32][64]; [192] */
  const float *fw, *fb;       /* [8][64]: move rows 0-4, bomb 5-6, critic 7; [8] */
  const uint8_t* move_mask;
  const uint8_t* bomb_mask;
  const float* uniforms;      /* [B][out_slots][2] (move, bomb) or NULL = Philox */
  int64_t* actions;           /* [B][out_slots][2] or NULL */
  int8_t* actions_i8;         /* [B][out_slots][2] or NULL */
  float* logp_out;            /* [B][out_slots] or NULL */
  float* value_out;           /* [B][out_slots] or NULL */
  float* logits_out;          /* [B][out_slots][8]: 5 move, 2 bomb, value; or NULL */
  uint16_t* workspace;        /* >= ceil(B * npid / 32) * 32 * QQT_CNN_WS_BYTES_PER_ITEM
                                 bytes, 16-byte aligned: the trunk's float16 hi / lo
                                 features, in blocks of 32 items */
  int64_t workspace_bytes;
} qqt_cnn_args;
int qqt_cnn_act(const qqt_cnn_args* args, void* stream);

/* Per-player features of the lstm arch (replaces sim/obs.py:243-340,
 * local_view_features, which the reference's collect loop calls each tick
 * for its lstm learner, train/ppo.py:227-231).  From the sim state and its
 * float16 observation: local = the 7x7 window of every channel around the
 * player's centre cell (zero outside the grid); rel = the P-1 opponents
 * (pos difference on axis 0, on axis 1, alive) then the bombs nearest in L1
 * distance (column offset, row offset, 0, 1; equal distances in ascending
 * cell index; slots past the last bomb hold the offsets of the lowest-index
 * remaining cells with flag 0); glob = t/max_steps, hp/max_hp, danger at the
 * centre cell, bombs/max_bombs, fuse sum/(max_bombs*fuse).  Outputs are
 * float16, rows of p_out players per env, `*_stride` elements apart (so a
 * call can write straight into a rollout buffer's slot). */
typedef struct qqt_lstm_feat_args {
  int32_t n_envs;
  int32_t p_out;              /* 1: player 0 only (only_p0=True), or n_players */
  const int32_t* cells;       /* sim state, layout above */
  const int32_t* players;
  const int32_t* envs;
  const uint16_t* obs;        /* [N][5P+4][H][W] float16 of the same state */
  uint16_t* local;            /* per env [p_out][C][7][7] */
  uint16_t* rel;              /* per env [p_out][10][6] */
  uint16_t* glob;             /* per env [p_out][5] */
  int64_t local_stride, rel_stride, glob_stride;   /* elements between envs */
} qqt_lstm_feat_args;
int qqt_lstm_features(const qqt_sim_config* cfg, const qqt_lstm_feat_args* args, void* stream);

/* lstm actor/critic step (replaces ActorCritic.act / forward with arch
 * "lstm", train/model.py:103-120, 176-185, 198-214, 230-245): per row the
 * 7x7 conv trunk (C->32->64, 2x2 max pool, Linear 576->128), the rel and glob
 * MLPs, the 256-wide fusion layer, one LSTM step (hidden 128) and the heads,
 * then masked sampling (the same Philox draws and sampler as qqt_mlp_act).
 * Every product runs on the float16 MFMA (v_mfma_f32_16x16x32_f16) with the
 * float32 operands split into float16 hi + lo, taken as hi*hi + hi*lo +
 * lo*hi with float32 accumulation: within 5e-6 of the float32 reference
 * module (measured 4.3e-6 over a 12-frame sequence).  The split saturates
 * at float16's 65504: larger activations stay finite, with the remainder
 * carried at float16 precision.  Row r belongs to env
 * r / rows_per_env and player (rows_per_env == 1 ? pid0 : r % rows_per_env).
 * h and c are read (zero for rows of envs with reset[env] != 0) and
 * overwritten with the new state. */
typedef struct qqt_lstm_args {
  int32_t batch;              /* rows B */
  int32_t c_in;               /* observation channels C of the local windows (<= 14) */
  int32_t rows_per_env;       /* 1 or P */
  int32_t pid0;
  int32_t sample;             /* 1: draw actions (needs masks) */
  uint64_t seed;              /* Philox key of the policy uniforms */
  uint32_t tick;              /* counter word of the policy uniforms */
  const uint16_t* local;      /* [B] rows of [C][7][7] float16 */
  const uint16_t* rel;        /* [B] rows of [10][6] */
  const uint16_t* glob;       /* [B] rows of [5] */
  int64_t local_stride, rel_stride, glob_stride;   /* elements between rows */
  const float* params;        /* packed parameters (qqtsim/policy.py pack_lstm, QQT_LSTM_PARAMS floats) */
  float* h;                   /* [B][128] hidden state in / out */
  float* c;                   /* [B][128] cell state in / out */
  const uint8_t* reset;       /* [envs] or NULL */
  const uint8_t* move_mask;   /* row r at r * mm_row_stride, 5 bytes */
  const uint8_t* bomb_mask;   /* row r at r * bm_row_stride, 2 bytes */
  int32_t mm_row_stride, bm_row_stride;
  const float* uniforms;      /* [B][2] (move, bomb) or NULL = Philox */
  int32_t out_stride, out_slot;   /* outputs of row r at slot r * out_stride + out_slot */
  int64_t* actions;           /* [slot][2] or NULL */
  int8_t* actions_i8;         /* [slot][2] or NULL */
  float* logp_out;            /* [slot] or NULL */
  float* value_out;           /* [slot] or NULL */
  float* logits_out;          /* [B][8]: 5 move, 2 bomb, value; or NULL */
} qqt_lstm_args;
#define QQT_LSTM_PARAMS 378880
int qqt_lstm_act(const qqt_lstm_args* args, void* stream);

/* Dispatch timing for benchmark harnesses (no counterpart in the reference:
 * its bench times whole steps with host clocks).  qqt_timing_arm(n) times
 * the next n kernel launches made through this library: each records a
 * start/stop event pair on its own dispatch packet (hipExtLaunchKernel), so
 * the pair spans that kernel alone.  qqt_timing_collect waits for the timed
 * launches, writes per kernel kind (QQT_KERNEL_*, n_kinds entries) the
 * summed duration in ms and the number of timed launches, and disarms.  At
 * most 4096 launches are timed between collects.  Allocates no device
 * memory (the event pool is created by the first arm). */
enum { QQT_KERNEL_TICK = 0, QQT_KERNEL_MLP = 1, QQT_KERNEL_BOT = 2, QQT_KERNEL_REACH = 3,
       QQT_KERNEL_GAE = 4, QQT_KERNEL_L1GRAD = 5, QQT_KERNEL_PPO = 6, QQT_KERNEL_CNN = 7 /* trunk */,
       QQT_KERNEL_LSTM_FEAT = 8, QQT_KERNEL_LSTM = 9, QQT_KERNEL_CNN_HEAD = 10,
       QQT_KERNEL_KINDS = 11 };
int qqt_timing_arm(int32_t launches);
int qqt_timing_collect(double* ms, int32_t* count, int32_t n_kinds);

#ifdef __cplusplus
}
#endif

#endif /* QQT_HIP_H */
