/* sbenv: MI355X-native batched Smart Buildings environment step.
 *
 * C ABI of the PufferLib "ocean" env binding for the Smart Buildings env, GPU
 * backend (PUF_BACKEND == PUF_GPU). Every entry point below replaces the
 * reference function of the same name:
 *
 *   puf_vec_create  complete_port/gpu/smart_buildings.cu:2497 (impl), :3311 (export)
 *   puf_bind_stream complete_port/gpu/smart_buildings.cu:2887, :3314
 *   puf_init        complete_port/gpu/smart_buildings.cu:2891, :3315
 *                   (CPU env: complete_port/pufferlib_cpu_env.h:293)
 *   puf_reset       complete_port/gpu/smart_buildings.cu:2896, :3316
 *                   (CPU env: complete_port/pufferlib_cpu_env.h:187)
 *   puf_step        complete_port/gpu/smart_buildings.cu:2979, :3317
 *                   (CPU env: complete_port/pufferlib_cpu_env.h:211)
 *   puf_render      complete_port/gpu/smart_buildings.cu:3318 (no-op)
 *   puf_close       complete_port/gpu/smart_buildings.cu:3319
 *   puf_log         complete_port/gpu/smart_buildings.cu:3320
 *                   (CPU env keys: complete_port/pufferlib_cpu_env.h:284-291)
 *   puf_live_log    complete_port/gpu/smart_buildings.cu:3069, :3321
 *   puf_mask_init   complete_port/gpu/smart_buildings.cu:3230, :3322
 *
 * Buffers: the trainer owns obs [n x SB_OBS] f32, actions [n x (SB_CONT+SB_DISC)]
 * f32, rewards [n] f32 and terminals [n] f32, all device memory; the env writes
 * them in place. All device work runs on the stream given to puf_bind_stream
 * (hipStream_t; NULL = the null stream) and puf_step neither allocates nor
 * synchronises, so it can be captured in a hipGraph. Errors print to stderr and
 * abort(), as the reference does (pufferlib_cpu_env.h:189-190, 316-321).
 *
 * PufferLib's own pufferenv.h is not part of the reference; the Agent / Dict
 * layouts here carry the fields the reference env uses (observations, actions,
 * rewards, terminals, action_mask, policy; dict_find / dict_set) and are this
 * build's stated assumption about that header.
 */
#ifndef SBENV_H
#define SBENV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SB_OBS 1024
/* Action row: SB_CONT continuous heads, then SB_DISC discrete ones. Built with
 * -DSB_CONT_BIG (libsbenv_big.so) the row holds 320 continuous heads, for
 * buildings with more than 256 continuous actions, as the reference GPU env
 * built with SB_CONT_BIG (complete_port/gpu/smart_buildings.cu:35-61); a
 * trainer compiled against one layout links the matching library. */
#ifdef SB_CONT_BIG
#define SB_CONT 320
#else
#define SB_CONT 256
#endif
#define SB_DISC 16
#define SB_ACT (SB_CONT + SB_DISC)
#define SB_MASK_WIDTH (SB_CONT + 2 * SB_DISC)
#define OBS_SIZE SB_OBS
#define NUM_ATNS SB_ACT

typedef float obs_t;

/* Episode log of the reference GPU env this library replaces,
 * complete_port/gpu/smart_buildings.cu:101-115 (n is the last field, as the
 * trainer's log aggregation requires). Filled when an episode ends
 * (finalize_k, :1936-2047): the trainer may clear it between steps, so the
 * running sums stay on the device. Every field but n is a sum over the
 * episodes logged since the last clear: perf and score the episode's mean
 * reward, episode_return and episode_length, the episode means of the
 * per-step mean zone deviation from the comfort band (comfort_dev_K), of the
 * fraction of zones outside it (out_of_band_frac), of the normalized
 * productivity term, energy cost and carbon, the episode's worst zone
 * deviation (worst_dev_K), and its electricity and gas kWh. */
typedef struct Log {
    float perf;
    float score;
    float episode_return;
    float episode_length;
    float comfort_dev_K;
    float worst_dev_K;
    float out_of_band_frac;
    float productivity;
    float energy_cost_norm;
    float carbon_norm;
    float elec_kwh;
    float gas_kwh;
    float n;
} Log;

typedef struct Agent {
    obs_t* observations;
    float* actions;
    float* rewards;
    float* terminals;
    unsigned char* action_mask;
    int policy;
} Agent;

/* complete_port/pufferlib_cpu_env.h:91-121 (Log first, no pointers into Env). */
typedef struct Env {
    Log log;
    Agent agents[1];
    int num_agents;
    int tag;
    int boundary_reached;
    int step;
    int max_steps;
    int start_offset;
    int n_act, n_cont, n_disc;
    int loaded;
    unsigned int rng;
    int seed;
    int index;          /* position in the vec */
    void* vec;          /* owning vec (opaque) */
} Env;

typedef struct DictItem {
    const char* key;
    float value;
    const char* str;
} DictItem;

typedef struct Dict {
    DictItem* items;
    int size;
    int capacity;
} Dict;

/* Dict helpers with the semantics the reference env relies on. */
DictItem* dict_find(Dict* d, const char* key);
void dict_set(Dict* d, const char* key, float value);

/* ---- PufferLib env ABI ----
 * puf_vec_create kwargs ([env] section): blob | blob_dir (or SB_BLOB_DIR),
 * groups, max_steps, reward_scale (<= 0 means 1), desync (1: each env's first
 * episode ends at a hashed step in [1, episode length] and stays out of the
 * episode log; smart_buildings.cu:2583-2590, 2808-2815, 1990-1993), and the
 * canonical / residual / res_scale / res_dscale / guard_d0 / guard_d1 / guard_hot
 * (the canonical policy interface over the on-device pid_water base, see
 * sbx_canon_state), and the reference keys this env does not implement,
 * accepted only at 0 (random_start, rew_norm, rew_center, plant_pair,
 * comfort_shape, zone_*, ahu_critic, interleave, prestart_explore, probe).
 * Extras: start_offsets (1: every env starts its episodes at its own seeded
 * calendar offset, start_seed), shard_base (this vec's first env index in a
 * batch sharded over several vecs), per_env_seed (occupancy / convection seed
 * + index within the scenario, default 1), solver, envs_per_block,
 * trace_air (1: each step also stores every env's air side, air_g and air_T
 * as the reference core's state holds them, so sbx_env_state reports them;
 * without it the RC scenarios' snapshots carry NaN there). The Log
 * is filled at episode ends (the reference GPU env's form); the key log_at_end
 * is accepted at 1 only (the per-step Log of earlier versions is gone). */
Env* puf_vec_create(int n, Dict* kwargs, obs_t* observations, float* actions,
                    float* rewards, float* terminals);
/* NULL binds the null stream (the binding before any call); the reference
 * ignores NULL instead, which would leave a stale stream bound. */
void puf_bind_stream(void* stream /* hipStream_t */);
void puf_init(Env* env, Dict* kwargs);
void puf_reset(Env* envs);
void puf_step(Env* envs);
void puf_render(Env* env);
void puf_close(Env* envs);
/* Every Log field under its name (smart_buildings.cu:3044-3066). */
void puf_log(Log* log, Dict* out);
/* Totals since the previous call (a device reduction, then one sync):
 * env_steps, episodes, reward_mean over every env, and, when the vec holds
 * more than one scenario, scenario/<name>/reward and
 * scenario/<name>/comfort_dev_K, the scenario's mean reward and mean zone
 * deviation per env-step of the window (smart_buildings.cu:3069-3100; <name>
 * is the blob's file name without .sbb). */
void puf_live_log(Env* envs, Dict* out);
void puf_mask_init(unsigned char* mask, int width, int nagents);

/* ---- extras (no reference counterpart) ---- */

/* Writes one Beta(2,2) action row per env into the vec's action buffer on the
 * bound stream: Philox4x32-10 keyed by `seed`, counter (env, step, slot, 0),
 * median of three U(0,1); continuous slots get 2x-1, discrete slots x > 0.5.
 * The synthetic stand-in for a policy in benchmarks and parity tests. */
void sbx_gen_actions(Env* envs, uint64_t seed, uint32_t step);

typedef struct SbxVecInfo {
    int n_envs;
    int n_layouts;
    int n_scenarios;
    int block;              /* threads per workgroup (128 per env: two wavefronts) */
    int lds_bytes;          /* dynamic LDS per workgroup */
    int max_nodes;
    double bytes_per_step;  /* algorithmic HBM bytes of one puf_step (all envs): per env the
                               persistent state read and written (T, per-VAV and per-AHU
                               state, plant scalars, occupancy; interior mass where present),
                               the action row, the observation prefix, reward and terminal */
    double flops_per_step;  /* fp64 flops of one puf_step's solves (all envs) */
    int envs_per_block;     /* envs sharing a workgroup (two wavefronts each) */
    double record_bytes_per_step;   /* what the kernel's per-env record round trip moves for
                                       the same (its record image is wider than the state) */
} SbxVecInfo;
void sbx_vec_info(Env* envs, SbxVecInfo* out);

/* Synchronous snapshot of env `i` in the oracle's state order (temp, mass,
 * VAV damper/reheat/ratio/sensing, AHU flow/sat/recirc/fan, air_g, air_T,
 * occupancy, boiler current/return/setpoint, pump head, calendar index),
 * followed by two extras: the f64 sum of rewards and the number of steps since
 * puf_reset. On RC scenarios air_g / air_T are the last step's under the
 * kwarg trace_air (zero before the first step) and NaN without it; field
 * scenarios keep them in their records. Returns the number of doubles written
 * (<= cap), or -1. */
int sbx_env_state(Env* envs, int i, double* out, int cap);

/* Step-kernel timer on the bound stream: on = p > 0 clears it and makes every
 * p-th following puf_step (the first, then every p launches) record a HIP
 * event pair around its kernel launch (up to 16384 pairs); on = 0 stops it,
 * synchronises and returns the mean per-launch duration in microseconds of the
 * launches timed (*count of them). */
double sbx_kernel_timer(Env* envs, int on, int* count);

/* Launches the step kernel `iters` times back to back between two HIP events
 * on the bound stream and returns the elapsed milliseconds (synchronises). */
float sbx_time_step(Env* envs, int iters);

/* puf_step with the step's action rows read from `actions` (device, n x
 * NUM_ATNS floats, same layout as the bound buffer) instead of the buffer bound
 * at puf_vec_create; the bound buffer is not touched. For drivers that keep a
 * bank of pre-drawn action rows resident (the benchmark). No counterpart in the
 * reference. Returns 0, or -1 for a null pointer. Asynchronous on the bound
 * stream, capturable. */
int sbx_step_actions(Env* envs, const float* actions);

/* Runs one step with per-phase wall-clock stamps and reports, for phases
 * 0..n-1 (load, decode, HVAC pre, solve setup, solve, solve epilogue, post,
 * observation, occupancy, reward, bookkeeping, store), the mean and max
 * duration over workgroups in microseconds. Advances the envs by one step and
 * synchronises. Returns the number of phases written. */
int sbx_phase_times(Env* envs, double* mean_us, double* max_us, int n_phases);

/* Runs one step and copies the raw wall-clock stamps of every env (32 per
 * env, env-major; the phases above are stamps 0..12, unused stamps read 0).
 * Returns the number written, or -1 when cap is below 32 * n. */
int sbx_phase_stamps(Env* envs, unsigned long long* out, int cap);

/* Runs one step recording the shader-clock duration of every solve pass of
 * env `env`'s workgroup (for a layout on the relaxation solver: the setup,
 * then every sweep). Returns the number of entries written (<= cap). */
int sbx_pass_times(Env* envs, int env, long long* cycles, int cap);

/* Field solver of env i's layout and its counters: out[0] solver (0 LU plan,
 * 1 point relaxation, 2 block relaxation), out[1] the certified contraction
 * bound rho (relaxation; 0
 * otherwise), out[2] relaxation sweeps of the env's last step, out[3] steps of
 * the env that stopped at the sweep cap (64) without meeting the error bound.
 * The solver is chosen per vec by kwargs "solver": "auto" (default: block
 * relaxation where it is certified — A an M-matrix, blocks of at most 3 nodes,
 * at most 128 blocks and 8 off-block entries per block, rho <= 0.5 — else point
 * relaxation where certified — rho <= 0.5, at most 256 solved cells and 8
 * off-diagonal entries per row — else the LU plan), "relax" (the same without
 * the LU fallback), "point" or "lu". Returns 4, or -1. Synchronous. */
int sbx_solve_info(Env* envs, int i, double* out);

/* Shared-policy rollout step (the reference trainer's
 * policy forward runs between env steps). fp32 MLP on MFMA over every env's
 * observation row: h1 = tanh(obs W1 + b1), h2 = tanh(h1 W2 + b2),
 * y = h2 W3 + b3 = (u[256], v[256], ud[16], vd[16]); head j draws
 * x ~ Beta(softplus(u_j) + f, softplus(v_j) + f) (f = beta_floor; two
 * Marsaglia-Tsang gamma draws on Philox4x32-10 keyed by seed, counter (env,
 * step, 2j or 2j + 1, 1 + attempt), a shape below 1 boosted as
 * G(k + 1) U^(1/k)); continuous heads write 2x - 1, discrete heads x > 0.5 into the
 * vec's action rows (0 past the env's n_cont / n_disc). Weights are caller-owned
 * device memory, row-major [in][out]: W1 [1024][128], W2 [128][128],
 * W3 [128][544], biases [128], [128], [544]. sbx_policy_bind stores them and
 * allocates the activations (call it outside graph capture); sbx_policy_act
 * launches on the bound stream and allocates nothing. sbx_policy_heads copies
 * y of the last sbx_policy_act to host (synchronous). Return 0 / count, or -1. */
#define SBX_POLICY_HIDDEN 128
#define SBX_POLICY_HEADS (2 * SB_ACT)
typedef struct SbxPolicy {
    const float* w1;
    const float* b1;
    const float* w2;
    const float* b2;
    const float* w3;
    const float* b3;
    float beta_floor;   /* shape floor f: a = softplus(u) + f (the reference's policy.beta_floor);
                           1 gives shapes >= 1, below 1 shapes may fall under 1 (boosted gamma
                           draws); finite and > 0, as the reference trainer requires
                           (pufferlib_core.diff:5204-5208); -1 otherwise */
} SbxPolicy;
int sbx_policy_bind(Env* envs, const SbxPolicy* p);
int sbx_policy_act(Env* envs, uint64_t seed, uint32_t step);
/* sbx_policy_act for callers that cannot allocate device memory (code under
 * hipGraph capture, tight serving loops, harnesses that forbid hipMalloc); no
 * counterpart in the reference. Needs no sbx_policy_bind: the weights come with
 * the call, and the activations live in a file-scope device array of the
 * library (12.5 MiB per GPU, held until the process ends) that fits at most
 * SBX_NOALLOC_MAX_ENVS envs; a larger vec is rejected (-1, message in
 * sbx_last_error). Same kernels and action rows as sbx_policy_act; launches on
 * the bound stream, no allocation, no synchronisation. Every call on one GPU
 * shares that array: calls that overlap on one GPU race. Returns 0, or -1. */
#define SBX_NOALLOC_MAX_ENVS 4096
int sbx_policy_act_noalloc(Env* envs, const SbxPolicy* p, uint64_t seed, uint32_t step);
int sbx_policy_heads(Env* envs, float* out, int cap);

/* Rollout-buffer side of the Beta heads (complete_port/patches/
 * pufferlib_core.diff:944-1000, beta_continuous_head; the trainer stores each
 * draw with its log-probability and entropy). With a = softplus(u) + f,
 * b = softplus(v) + f (float, as the sampler maps them; f the bound policy's
 * beta_floor), a head's draw x has
 * log p = (a - 1) log x + (b - 1) log(1 - x) - ln B(a, b) (x clamped to
 * [2^-24, 1 - 2^-24]) and entropy H = ln B(a, b) - (a - 1) psi(a) - (b - 1) psi(b)
 * + (a + b - 2) psi(a + b), evaluated in f64 and stored as float.
 * sbx_policy_act_logp: sbx_policy_act (same draws and action rows) that also
 * writes draws [n][272] (each used head's x in (0, 1), 0 elsewhere) and the
 * per-env sums over used heads logp [n] and entropy [n] (fixed summation
 * order). sbx_beta_eval: the same sums for given heads y [n][544] (the layout of
 * sbx_policy_heads) and draws [n][272], and, when grad is not null, grad
 * [n][4][272] = d log p / du, d log p / dv, d H / du, d H / dv per head (0 for
 * unused heads). Continuous head h reads u = y[h], v = y[256 + h]; discrete
 * head d (column 256 + d) reads u = y[512 + d], v = y[528 + d]. Device
 * pointers, caller-owned; both need sbx_policy_bind first (its scratch), launch
 * on the bound stream and allocate nothing. Return 0, or -1. */
int sbx_policy_act_logp(Env* envs, uint64_t seed, uint32_t step, float* draws, float* logp, float* entropy);
int sbx_beta_eval(Env* envs, const float* y, const float* draws, float* logp, float* entropy, float* grad);

/* PPO side of the Beta heads, one minibatch row per env (the reference's PPO
 * loss, complete_port/patches/pufferlib_core.diff:1205-1252, with its
 * ratio_per_dim, :539-543, and beta_kl, :1008-1014). Inputs (device, caller
 * owned): the new and the old policy's heads y_new, y_old [n][544] (the layout
 * of sbx_policy_heads), the rollout draws [n][272], the stored log-probability
 * logp_old [n] and advantages adv [n]. Over the env's D used heads, summed in
 * f64 in a fixed order: logp = sum log p_new(x), H = sum of the new heads'
 * entropies, KL = sum KL(old head || new head). lr = (logp - logp_old) / D
 * when ratio_per_dim (the geometric-mean ratio) else logp - logp_old,
 * non-finite -> 0, clamped to [-20, 20]; r = exp(lr);
 * pg = s max(-A r, -A clamp(r, 1 - clip, 1 + clip)), s = D when ratio_per_dim
 * else 1. out [n][6] = logp, H, KL, r, pg, lr. grad [n][2][272] (or NULL): the
 * derivative of pg - ent_coef H in each used head's u and v (0 elsewhere), with
 * d pg / d logp = -A r, or 0 where the clipped term is the larger and r lies
 * outside the clip range. Launches on the bound stream, allocates nothing.
 * Returns 0, or -1. */
typedef struct SbxPpo {
    float clip_coef;
    float ent_coef;
    int ratio_per_dim;
    float beta_floor;   /* finite and > 0 (as SbxPolicy.beta_floor) */
} SbxPpo;
int sbx_ppo_beta(Env* envs, const float* y_new, const float* y_old, const float* draws, const float* logp_old,
                 const float* adv, const SbxPpo* args, float* out, float* grad);

/* The heads' Beta sampler alone: out[i] ~ Beta(alpha[i], beta[i]) for device
 * arrays of n floats (alpha, beta > 0), counter (i, 0, 0 or 1, 1 + attempt),
 * on `stream` (hipStream_t; NULL = the null stream). Leaves the stream bound
 * by puf_bind_stream alone. Returns 0, or -1. */
int sbx_beta_sample(const float* alpha, const float* beta, float* out, int n, uint64_t seed, void* stream);

/* Canonical interface (kwargs canonical = 1, residual, res_scale, res_dscale,
 * guard_d0/d1/hot; complete_port/gpu/sb_gpu_base.inc): the trainer's rows hold
 * the canonical observation (983 floats) and canonical action heads (219,
 * SBC_ACT; Env.n_cont reads 219, n_disc 0); the env keeps its own observation
 * row internally and runs the pid_water base controller on it. Synchronous
 * copy of env i's own observation row (SB_OBS floats), the base proposal per
 * native action (SB_ACT floats) and the PID state (18 doubles: integral,
 * previous error per AHU slot); each pointer may be NULL. Returns the env's
 * native action count, or -1 (not canonical). */
int sbx_canon_state(Env* envs, int i, float* raw_obs, float* base, double* pid);

/* Scenario of env i (index into the sorted, round-robin ordered blob list),
 * its calendar start offset and occupancy seed. */
int sbx_env_meta(Env* envs, int i, int* scenario, int* start, uint32_t* occ_seed);
const char* sbx_scenario_path(Env* envs, int scenario);

/* Host-side solve plan of one blob's layout (no GPU needed): the level
 * schedule the step kernel runs for the numeric LU of A + diag(g) plus both
 * triangular solves. Slot 0 holds 0.0, slot 1 is a write sink, slot 2 holds
 * 1.0; inv_base.. hold pivot reciprocals. Pass p is pass_info[4p..4p+3] =
 * {hdr_off, word_off, nact | maxcnt << 8 | has_pivot << 16 | lgmax << 17, 0}:
 * lane l < nact holds hdr[hdr_off + l] = target | mul << 16 | inv_target << 32
 * | flags << 48 (flags = log2 segment width | leader << 3 | count << 4) and
 * terms words[word_off + l * stride + m], stride = maxcnt rounded up to 4
 * ((0, 0) past the count); a task's segment of lanes computes
 * slot[target] = (slot[target] - sum_m slot[a_m] * slot[b_m]) * slot[mul],
 * then, when has_pivot, slot[inv_target] = 1 / slot[target]. A term word is
 * a_m | b_m << 16, or with term_bits 12 three factors (below).
 * Arrays are owned by the library until sbx_plan_free. */
typedef struct SbxPlan {
    int n;               /* unknowns */
    int width;           /* lanes per pass */
    int n_slots;         /* LDS value slots: 0 = zero, 1 = sink, LU, vector */
    int vec_base;        /* first vector slot */
    int inv_base;        /* first pivot-reciprocal slot */
    int n_pass;
    int n_levels;
    int n_tasks;
    int kmax;            /* max terms per task */
    long long n_pairs;   /* multiply-subtract terms */
    int n_hdr, n_words;
    const int* pass_info;        /* [n_pass * 4] */
    const uint64_t* hdr;         /* [n_hdr] */
    const uint32_t* words;       /* [n_words]: a | b << 16 */
    const double* slot_init;     /* [n_slots] A values at LU slots, 0 elsewhere */
    const int* pos;              /* [n] node -> permuted position */
    const int* air_slot;         /* [k] LU slot of the coupled air diagonal */
    const int* air_node;         /* [k] node of coupled column c */
    int k;
    /* relaxation form: rows padded to rx_rows; entry m of row i at m * rx_rows + i
     * of rx_val / rx_col, (0.0, 0) past the row; x_i <- (b_i - sum_m rx_val *
     * x[rx_col]) / (rx_diag_i + g of air column rx_air_i, if >= 0) */
    int rx_ok;                   /* 1 when the relaxation form is certified */
    int rx_rows, rx_terms_max, rx_terms;
    double rx_rho;               /* max_i sum_j |a_ij| / a_ii */
    const double* rx_diag;       /* [rx_rows] */
    const int* rx_air;           /* [rx_rows] */
    const double* rx_val;        /* [rx_terms_max * rx_rows] */
    const int* rx_col;           /* [rx_terms_max * rx_rows] */
    /* block-Jacobi form: blocks of at most bx_rows nodes; lane l owns blocks l
     * and l + 64 (block slot q < bx_slots); tables lane-minor (64 lanes):
     * bx_row / bx_diag / bx_air at (q * bx_rows + p) * 64 + l (node or -1, a_ii,
     * air column or -1), bx_in at ((q * bx_rows + p) * bx_rows + p2) * 64 + l
     * (a(row p, row p2), 0 on p == p2), and the block's off-block entries
     * bx_val / bx_col / bx_trow at (q * bx_terms_max + t) * 64 + l (value,
     * column, row within the block; (0.0, 0, 0) padding) */
    int bx_ok;
    int bx_rows, bx_slots, bx_terms_max, bx_terms, bx_blocks;
    double bx_rho;               /* max_i sum_j (|A_BB^-1| |A_BO|)_ij */
    const int* bx_row;
    const double* bx_diag;
    const int* bx_air;
    const double* bx_in;
    const double* bx_val;
    const int* bx_col;
    const int* bx_trow;
    /* term word format: 16 = a | b << 16 as above; 12 = a | b << 12 | v << 24,
     * the product slot[a] * slot[scale_base + v] * slot[b] (slot scale_base
     * holds 1.0, scale_base + 1 + k the reciprocal of pivot k = inv_base + k),
     * used where n <= 255 and n_slots <= 4096: L is then stored unscaled
     * (L[i][k] * U[k][k]) and its readers multiply by the reciprocal */
    int term_bits;
    int scale_base;
} SbxPlan;
int sbx_plan_layout(const char* blob_path, int width, SbxPlan* out);
void sbx_plan_free(SbxPlan* p);

/* ---- Building-scale field step ------------------------------------------
 * The reference core's FDM step (complete_port/csim/sb_fdm.h:60-68,
 * sb_fdm_step_batch; sb_fdm.c:142-270) for G envs that share one blob's baked
 * factorization, on the device: forcing, the L and U sweeps of the SuperLU
 * factors, the air-side correction (sensed dots, the dense k x k solve, the
 * applied heat, a second solve), interior mass and the field. Results are
 * those of G sequential sb_fdm_step calls (bit for bit with SBX_FDM_EXACT,
 * to rounding otherwise). The blob needs only
 * the field sections (grid, solved, capacitance_rate, dirichlet_conductance,
 * mass_*, temp_init, horizontal, vertical, solver_conductivity,
 * ambient_face_areas_0/1, lu_L/lu_U/lu_perm_r/lu_perm_c, applied, sensed).
 * Envs are grouped in blocks of envs_per_block lanes (a power of two up to
 * 64); each block runs every level of a factor on one workgroup. */
typedef struct SbxFdm SbxFdm;
typedef struct {
    int n_cvs, n_solved, k;       /* cells, solved cells, air-side columns */
    int n_envs, envs_per_block, n_blocks;
    int levels_l, levels_u;       /* level-schedule depth of the two sweeps */
    long long nnz_l, nnz_u;       /* off-diagonal factor entries */
    double bytes_per_step;        /* algorithmic HBM bytes of one batched step */
    double flops_per_step;        /* multiply-adds x 2 of the solves and the air-side combination */
    int tail_rows_l, tail_rows_u;       /* rows of each sweep's LDS run (0: exact mode) */
    int tail_levels_l, tail_levels_u;   /* levels of the LDS run */
    int chunked_levels_l, chunked_levels_u;   /* levels after it solved chunked from HBM */
} SbxFdmInfo;
/* Flags of sbx_fdm_open. Default: each sweep's longest run of narrow levels
 * (at most 64 rows each: the separators at the top of the elimination tree,
 * as many as fit) runs with its rows in LDS, and the levels after it with
 * each row's terms spread over lanes; row sums are formed in another order,
 * so results agree with the reference to rounding, far inside 1e-9
 * relative. SBX_FDM_EXACT: every level from HBM in the reference's order,
 * bit-identical results. envs_per_block 0 picks 1 (default; 2 when there
 * are more envs than the GPU has compute units) or up to 64 (exact). The default mode also takes the air-side correction from the
 * responses of the applied columns (sbx_fdm_air_responses) instead of a
 * second solve per step. */
#define SBX_FDM_EXACT 1
/* sb_fdm_init for every env: the blob's initial fields, S = sensed A^-1 applied
 * (solved on the device, in the reference's order). NULL on error
 * (sbx_last_error). */
SbxFdm* sbx_fdm_open(const char* blob_path, int n_envs, int envs_per_block, int flags);
void sbx_fdm_close(SbxFdm* f);
int sbx_fdm_info(const SbxFdm* f, SbxFdmInfo* out);
/* One step of every env on `stream` (asynchronous). Device arrays, env-major
 * like the reference's per-env arguments: input_q [G][n_cvs] (heat per cell),
 * ambient and h [G] (ambient temperature, convection coefficient), air_g and
 * air_T [G][k] (air-side conductance and supply temperature per coupled
 * column; an env whose k conductances are all 0 has no air side this step). */
int sbx_fdm_step(SbxFdm* f, const double* input_q, const double* ambient, const double* h, const double* air_g,
                 const double* air_T, void* stream);
/* Every env back to the blob's initial fields. */
int sbx_fdm_reset(SbxFdm* f, void* stream);
/* Host arrays, env-major: temp [G][n_cvs], mass_temp [G][n_solved]. Synchronise. */
int sbx_fdm_get_state(SbxFdm* f, double* temp, double* mass_temp);
int sbx_fdm_set_state(SbxFdm* f, const double* temp, const double* mass_temp);
/* S [k][k] (host). */
int sbx_fdm_sensed_response(SbxFdm* f, double* out);
/* The default mode's air-side responses R [k][n_solved] (host): row j is
 * A^-1 applied_j by solved index, solved at open in the reference's order
 * (sb_fdm.c:104-108 solves the same columns for S). A step's air-side
 * correction (sb_fdm.c:171-178: the applied heat of the dense solve's q,
 * solved again) is then the combination sum_j q_j R[j] (linear in q: equal
 * to rounding). Returns 1 (and writes nothing) in exact mode, which solves
 * the correction as the reference does, or when k = 0. */
int sbx_fdm_air_responses(SbxFdm* f, double* out);
/* x = A^-1 b through the baked factors on the device (sb_lu_solve,
 * sb_lu.c:38-63), for n_rhs host columns b, x [n_rhs][n_solved]. */
int sbx_fdm_lu_solve(SbxFdm* f, const double* b, double* x, int n_rhs);

/* Message of the last failing sbx_* call. */
const char* sbx_last_error(void);
const char* sbx_version(void);
/* SB_CONT of this build (256, or 320 for libsbenv_big.so), so a binding can
 * check it loaded the library its action rows are laid out for. No
 * counterpart in the reference, whose layout is fixed at compile time. */
int sbx_cont_width(void);

#ifdef __cplusplus
}
#endif
#endif
