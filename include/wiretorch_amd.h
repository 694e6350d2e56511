/* wiretorch_amd.h — C-ABI of the MI355X (gfx950) conductance-LIF hot path.
 *
 * The reference (rory-bedford/wiretorch) drives this path from Python with Triton
 * launches; it has no C/C++ FFI of its own. Each entry point below replaces the
 * launches named in its comment (file:line in the reference), behind the reference's
 * unchanged Python contract `conductance/engine.py:71-89` (`simulate`) and its
 * autograd functions `_FeedforwardScan` (:444-474) / `_RecurrentRun` (:477-544).
 *
 * Conventions
 *  - All pointers are device pointers (hipMalloc / torch CUDA tensors) unless noted;
 *    sizes are int64_t. Nothing here allocates device memory or synchronises the host.
 *  - Layouts are the reference's (conductance/kernels.py:20-35):
 *      v (B,N) f32; g (B,2,S,N) f32 (component 0 = rise, 1 = decay); counter (B,N) i32;
 *      spikes/prob/v_saved (B,T,N) f32; G_saved (B,T,N,S) f32; held (B,T,N) i8;
 *      A (K,B,T,N) f32 (pathway activations, recurrent pathways first).
 *  - dt and surr_scale are device pointers to 0-d f32 tensors (no host sync).
 *  - Connectivity is passed compressed, by source (see wt_side): the reference's dense
 *    per-pathway rows (network.py:106-157) are converted by the host once per call.
 *  - Every entry point takes the hipStream_t to enqueue on and returns a hipError_t
 *    value as int (0 = success); invalid arguments return hipErrorInvalidValue (1)
 *    without launching.
 */
#ifndef WIRETORCH_AMD_H
#define WIRETORCH_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* wt_stream_t; /* a hipStream_t */

/* Per-neuron and per-synapse tables of one call (the reference's Physiology,
 * conductance/dynamics.py:56-92, padded: S <= WT_MAX_S). */
#define WT_MAX_S 8
#define WT_MAX_K 8
typedef struct {
  const float* theta;    /* (N,) */
  const float* U_reset;  /* (N,) */
  const float* E_L;      /* (N,) */
  const float* C_m;      /* (N,) */
  const float* beta;     /* (N,) */
  const int32_t* n_ref;  /* (N,) or NULL: no refractory period */
  const float* E_syn;    /* (S,) */
  const float* g_clip;   /* (S,) */
  const float* decay;    /* (2,S) */
  const float* jump;     /* (2,S) */
  const float* made;     /* (K,S) 0/1 */
  const float* scale;    /* (K,N) */
  const float* dt;       /* 0-d */
  const float* surr;     /* 0-d */
  /* The same per-neuron values deduplicated (used by wt_cond_run): rows of (theta,
   * U_reset, E_L, C_m, beta, n_ref, scale[0..K-1]). Without range_rows: n_types <= 256
   * rows, type_of (N,) picks a row. With range_rows (n_ranges, 256), the rows of the
   * target range of geometry range_n holding neuron n are range_rows[n / range_n][0 ..
   * n_types), n_types <= 256 then being the largest count over the ranges, and type_of[n]
   * indexes that list. */
  const float* types;
  const int32_t* type_of;
  int64_t n_types;
  const int32_t* range_rows;
  /* The NMDA Mg block (conductance/dynamics.py:110-129): each synapse type's current
   * scaled by B(v) = sigmoid(mg_a v - mg_lc), mg_lc = log(mg / mg_k), -inf for a type
   * without one; both (S,), or NULL when no type has a block. */
  const float* mg_a;
  const float* mg_lc;
  /* Spike-frequency adaptation (conductance/kernels.py:163-281, dynamics.py:116-143): a
   * neuron's adaptation conductance g_a (by E_adapt) adds g_a to the step's total
   * conductance and g_a (v - E_adapt) to its current, and after the step becomes g_a
   * adapt_decay + adapt s. All three (N,), or NULL when no neuron adapts. */
  const float* adapt;
  const float* adapt_decay;
  const float* E_adapt;
  int64_t N, S, K, K_rec;
} wt_tables;

/* One input side's connectivity, compressed by source and split by target range.
 * Source j's synapses onto targets in range r = [r*range_n, (r+1)*range_n) are
 * edges split[j*(R+1)+r] .. split[j*(R+1)+r+1]-1 (targets ascending); pathway[j] is
 * the pathway its activation feeds (-1: none). Built by wt_split_ranges. */
typedef struct {
  const int64_t* indptr;   /* (n_src+1,) */
  const int64_t* split;    /* (n_src, R+1) */
  const int32_t* targets;  /* (E,) */
  const float* weights;    /* (E,) */
  const int32_t* pathway;  /* (n_src,) */
  int64_t n_src;
} wt_side;

/* Launch geometry of wt_cond_run: groups*R workgroups; group g owns the trials
 * b = g, g+groups, ...; workgroup slot r of a group owns targets [r*range_n, ...);
 * range_n is a multiple of 32, and a workgroup owns at most 8192 (trial, neuron) items.
 * frac_bits: activations are accumulated exactly as int64 multiples of 2^-frac_bits.
 * bound: NULL, or a device pointer to the largest magnitude any activation can reach
 * (per-target sums of |weight| times the largest |input|); then the kernel derives
 * frac_bits itself, min(40, 51 - ceil(log2 bound)) (40 for a bound of 0), so the host
 * need not read the bound back, and the frac_bits field is ignored.
 * max_list: the per-workgroup event list, 1024 or 2048 entries (0 = the largest that
 * fits in LDS; 2048 needs at most 4096 items per workgroup and room beside the
 * accumulator). A step's events beyond the list are pushed in further rounds; results do
 * not depend on it. */
typedef struct {
  int64_t groups, R, range_n, frac_bits, max_list;
  const double* bound;
} wt_geometry;

/* wt_split_ranges — (re)build side->split for R target ranges of range_n targets
 * (binary search of each source's ascending targets). split: (n_src, R+1) int64. */
int wt_split_ranges(const int64_t* indptr, const int32_t* targets, int64_t n_src,
                    int64_t R, int64_t range_n, int64_t* split, wt_stream_t stream);

/* wt_cond_run — T steps of the conductance-LIF network, forward.
 * Replaces: conductance/kernels.py:159-289 scan_forward (feedforward networks,
 * K_rec = 0) and the per-step pair network_simulators/kernels.py:133-204
 * compact_spikes + conductance/kernels.py:572-700 recurrent_step launched by the host
 * loop conductance/engine.py:306-355 — here one persistent launch for all T steps.
 *   x (B,T,n_in) f32 input (or NULL with in_prob: on-device Poisson input); rec/ff:
 *   recurrent side (sources = the N neurons) and
 *   feedforward side (sources = the n_in input columns), rec may have n_src = 0.
 *   State v, g, counter is updated in place. Outputs: spikes (required); prob,
 *   v_saved, G_saved, held, A_saved (K,B,T,N) and the tracked v/I/g of trial track_b
 *   (-1: all) may each be NULL.
 *   scratch: device workspace of wt_cond_run_scratch_bytes bytes whose first
 *   wt_cond_run_scratch_zeroed bytes the caller zeroes before each launch. */
typedef struct {
  const float* x;
  int64_t B, T, n_in;
  float* v;
  float* g;
  int32_t* counter;
  float* spikes;
  float* prob;
  float* v_saved;
  float* G_saved;
  int8_t* held;
  float* A_saved;
  float* track_v;  /* (Bt,T,N) */
  float* track_I;  /* (Bt,T,N,S+1) */
  float* track_g;  /* (Bt,T,N,2,S) */
  int64_t track_b;
  /* On-device Poisson input instead of x (x NULL): channel j of trial b fires at step t
   * with probability in_prob[j] (n_in floats), drawn from Philox4x32-10 under key
   * in_seed at counter (j, in_t0 + t, b, 0) (see wt_poisson_fill); NULL: the input is x. */
  const float* in_prob;
  uint64_t in_seed;
  int64_t in_t0;
  /* With adaptation (tab.adapt): the adaptation conductances (B,N), updated in place;
   * a_saved (B,T,N) each step's g_a entering it, and track_a (Bt,T,N) g_a after it, may
   * be NULL. Without, all three are ignored. */
  float* adaptation;
  float* a_saved;
  float* track_a;
} wt_run_io;

/* wt_poisson_fill — materialise on-device Poisson input: x[b, t, j] = 1 if channel j of
 * trial b fires at absolute step t0 + t, else 0, (B, T, n_in) f32. A channel fires when
 * u < prob[j], u = (w >> 8) * 2^-24 with w the first word of Philox4x32-10 (Salmon et al.
 * 2011) of counter (j, t0 + t, b, 0) under key (seed low 32 bits, seed high 32 bits): the
 * stream wt_cond_run draws from with in_prob/in_seed/in_t0, which the host can replay.
 * Replaces the dense spike tensor the reference's Poisson dataset draws with torch.rand
 * (dataloaders/unsupervised.py:85-90). */
int wt_poisson_fill(const float* prob, int64_t n_in, uint64_t seed, int64_t t0, int64_t B,
                    int64_t T, float* x, wt_stream_t stream);

int64_t wt_cond_run_scratch_bytes(const wt_geometry* geo, int64_t B, int64_t T);
/* Leading bytes of the scratch that must be zero at each launch (the rest need not). */
int64_t wt_cond_run_scratch_zeroed(const wt_geometry* geo);
int wt_cond_run(const wt_tables* tab, const wt_side* rec, const wt_side* ff,
                const wt_geometry* geo, const wt_run_io* io, void* scratch,
                wt_stream_t stream);

/* wt_cond_run_noalloc — wt_cond_run for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. The workspace is a file-scope device array of
 * WT_NOALLOC_SCRATCH_BYTES bytes that every GPU the library runs on holds until the
 * process ends; the call allocates nothing (it zeroes what must start at zero with a
 * kernel of its own). Calls whose workspace (wt_cond_run_scratch_bytes) exceeds it return
 * hipErrorOutOfMemory (2) without launching: split T into chunks. Every call on one GPU
 * shares that GPU's array, so calls that overlap on one GPU (on different streams) race;
 * calls in one stream are safe. flags (device, 4 bytes, may be NULL) receives the run's
 * error flags, as the first word of wt_cond_run's scratch: 0, or nonzero when a group
 * barrier timed out. Arguments otherwise as wt_cond_run. */
#define WT_NOALLOC_SCRATCH_BYTES (64ll << 20)
int wt_cond_run_noalloc(const wt_tables* tab, const wt_side* rec, const wt_side* ff,
                        const wt_geometry* geo, const wt_run_io* io, uint32_t* flags,
                        wt_stream_t stream);

/* wt_cond_run_timed — wt_cond_run with per-workgroup wall-clock ticks (100 MHz) of each
 * phase of the step loop, as seen by the workgroup's first thread, added to
 * timing[wg * 8 + phase], phases: 0 bitmap and input loads + clears, 1 listing of the
 * fired sources, 2 range lookups + its own neuron update, 3 the wait for the rest of the
 * workgroup's update, 4 publication + unlisted events + barrier arrival, 5 barrier wait,
 * 6 appends to the event list, 7 scan + synapse push (+ further rounds). For profiling;
 * no counterpart in the reference. timing: (groups * R * 8) u64. Lean runs only: with
 * saved tensors, probabilities or tracking it returns hipErrorInvalidValue; it always
 * takes the 1024-entry event list (results do not depend on it). The timer is compiled
 * into kernels of their own, so that wt_cond_run's carry no check of it. */
int wt_cond_run_timed(const wt_tables* tab, const wt_side* rec, const wt_side* ff,
                      const wt_geometry* geo, const wt_run_io* io, void* scratch,
                      uint64_t* timing, wt_stream_t stream);

/* wt_cond_scan_backward — reverse-time adjoint of T steps whose activations A are
 * known (the recurrent activations treated as input).
 * Replaces: conductance/kernels.py:383-568 scan_backward (+ _membrane_adjoint
 * :315-379), launched by conductance/engine.py:358-383.
 *   Reads grad_spikes, grad_prob (may be NULL), spikes, v_saved, G_saved, held (NULL
 *   without refractory), A, g_init (NULL unless want_decay). Writes (each may be NULL
 *   when not wanted) grad_A (K,B,T,N), grad_scale partials (K,B,N), and per-(trial,
 *   neuron) partials: theta, U_reset, E_L, C_m, beta (B,N); E_syn (B,S,N);
 *   decay, jump (B,2,S,N). The caller sums the partials over trials. */
typedef struct {
  const float* grad_spikes;
  const float* grad_prob;
  const float* spikes;
  const float* v_saved;
  const float* G_saved;
  const int8_t* held;
  const float* A;
  const float* g_init;
  int64_t B, T;
  float* grad_A;
  float* grad_scale;
  float* grad_theta;
  float* grad_reset;
  float* grad_E_L;
  float* grad_C_m;
  float* grad_beta;
  float* grad_E_syn;
  float* grad_decay;
  float* grad_jump;
  /* With adaptation (tab.adapt): a_saved (B,T,N) from the forward, and the per-(trial,
   * neuron) partials (B,N) of adapt, adapt_decay and E_adapt (each may be NULL). */
  const float* a_saved;
  float* grad_adapt;
  float* grad_adapt_decay;
  float* grad_E_adapt;
  /* Optional, wt_cond_scan_backward only: dL/da written as rows instead of grad_A — row
   * k*N + n (pitch B*T_pad floats) holds pathway k's dL/da onto target n at b*T_pad + t,
   * T_pad a multiple of 16 and >= T (entries t >= T hold no value) — the layout that
   * wt_weight_gradient_by_target takes with grad_A NULL. grad_A is then not written. */
  float* grad_A_rows;
  int64_t T_pad;
} wt_backward_io;

int wt_cond_scan_backward(const wt_tables* tab, const wt_backward_io* io,
                          wt_stream_t stream);

/* wt_cond_recurrent_backward — the same adjoint when gradients also flow back through
 * the recurrent spikes (recurrent_gradients=True): per reverse step, dL/da of every
 * neuron, then R_j = sum over source j's synapses e of w_e * dL/da_k(j)[target e] added
 * to dL/ds_j before the surrogate. io as for wt_cond_scan_backward; rec is the
 * recurrent side (indptr, targets, weights, pathway; split unused), n_src == N.
 * scratch: wt_cond_recurrent_backward_scratch_bytes(S, K_rec, B, N) bytes, no zeroing
 * needed (adjoint state between the steps, the current step's dL/da and R).
 * Replaces: conductance/engine.py:386-438 _recurrent_backward — per step
 * conductance/kernels.py:704-823 inject_backward, network_simulators/engine.py:257-271
 * carry_to_sources, network_simulators/kernels.py:214-241 spike_backward. */
int64_t wt_cond_recurrent_backward_scratch_bytes(int64_t S, int64_t K_rec, int64_t B,
                                                 int64_t N);
int wt_cond_recurrent_backward(const wt_tables* tab, const wt_side* rec,
                               const wt_backward_io* io, void* scratch, wt_stream_t stream);

/* ===================================================================================
 * Rate networks (rate/dynamics.py): r = gain f(v - theta); a_k = r[rows_k] W_k (or the
 * input's columns times W_k); I <- decay I + (1 - decay) sum_k a_k jump_k;
 * v <- beta v + (1 - beta) sum_s sign_s I_s.
 * =================================================================================== */

/* Per-neuron and per-synapse tables of one call (rate/dynamics.py:72-92). */
typedef struct {
  const float* theta;          /* (N,) */
  const float* gain;           /* (N,) */
  const float* beta;           /* (N,) membrane decay per step */
  const int8_t* nonlinearity;  /* (N,) 0 relu, 1 softplus, 2 sigmoid, 3 tanh */
  const float* sign;           /* (S,) +1 excitatory, -1 inhibitory */
  const float* decay;          /* (S,) current decay per step */
  const float* jump;           /* (K, N, S) scale_k[n] * made_k[s] (rate/dynamics.py:95-97) */
  const float* made;           /* (K, S) */
  int64_t N, S, K, K_rec;
} wt_rate_tables;

/* The recurrent product's operand, zero-padded to whole 64 x 64 tiles: rows [0,
 * K_rec_pad) are the recurrent pathways' source neurons, each pathway a segment of whole
 * tiles, seg[g] = {first row, end row, pathway k, 0}, in pathway order. (The input
 * pathways' products x[:, :, rows] W_k come precomputed for the whole call, as
 * wt_rate_io.A_ff.) */
typedef struct {
  const void* W;          /* (K_rec_pad, N_pad), float32 or bfloat16 */
  const void* Wt;         /* (N_pad, K_rec_pad): W transposed, same dtype */
  void* rin;              /* [2][B_pad][K_rec_pad] rates of the step (zero-initialised) */
  const int32_t* rpos;    /* (N,) recurrent row of each neuron, or -1 */
  const int32_t* src_of;  /* (K_rec_pad,) neuron of each recurrent row, or -1 */
  int32_t seg[16][4];
  int64_t n_seg, B_pad, N_pad, K_rec_pad;
  int64_t dtype;          /* 0 float32, 1 bfloat16 (what W, Wt, rin hold) */
} wt_rate_operand;

typedef struct {
  int64_t B, T;
  float* v;             /* (B, N) in/out */
  float* I;             /* (B, S, N) in/out */
  float* out;           /* (B, T, N) rates */
  float* track_v;       /* (Bt, T, N) or null */
  float* track_I;       /* (Bt, T, N, S) or null */
  int64_t track_b;      /* -1: all trials */
  float* v_saved;       /* (B, T, N) voltage entering each step, or null */
  float* I_saved;       /* (B, T, N, S) currents entering each step, or null */
  float* target_saved;  /* (B, T, N, S) or null */
  float* A_saved;       /* (K, B, T, N) activations, or null */
  const float* A_ff;    /* (K - K_rec, B, T, N) input pathways' activations, float32 (null
                         * when K == K_rec) */
  float* split;         /* wt_rate_split_bytes scratch for the split product, or null */
} wt_rate_io;

/* wt_rate_forward — T steps of a rate network: per step one fused launch (MFMA product
 * of the rates with the weights, then currents, voltages and the next rates).
 * Replaces: rate/engine.py:157-300 (_Product, the per-step scan and recurrent kernels
 * rate/kernels.py:100-219). */
int wt_rate_forward(const wt_rate_tables* tab, const wt_rate_operand* op, const wt_rate_io* io,
                    wt_stream_t stream);

typedef struct {
  int64_t B, T;
  const float* grad_out;      /* (B, T, N) dL/d rates */
  const float* v_saved;       /* from the forward */
  const float* I_saved;
  const float* target_saved;
  const float* A_saved;
  const float* I_final;       /* (B, S, N) currents after the last step */
  float* lam_v;               /* (B, N) scratch, zeroed */
  float* lam_I;               /* (B, S, N) scratch, zeroed */
  float* d_rate;              /* (B, N) scratch, zeroed (recurrent networks) */
  void* gA_op;                /* (K_rec, B_pad, N_pad) scratch, zeroed, operand dtype */
  float* grad_A;              /* (K, B, T, N) out: dL/da */
  float* acc_theta;           /* (B, N) accumulated partials, or null */
  float* acc_gain;            /* (B, N) */
  float* acc_beta;            /* (B, N) */
  float* acc_decay;           /* (B, S, N) */
  float* acc_scale;           /* (K, B, N) */
} wt_rate_back_io;

/* wt_rate_backward — the reverse: per step dL/da_k from the currents' and voltages'
 * adjoints, then dL/dr = sum_k dL/da_k W_k^T (MFMA) into the rates' adjoint. Weight
 * and input gradients follow from grad_A by plain products on the host.
 * Replaces: rate/kernels.py:228-465, rate/engine.py:336-383 (_RecurrentRun.backward). */
int wt_rate_backward(const wt_rate_tables* tab, const wt_rate_operand* op,
                     const wt_rate_back_io* io, wt_stream_t stream);

/* wt_rate_split_bytes — scratch bytes (no zeroing needed) that let wt_rate_forward of a
 * drive with one recurrent pathway, every padded size a multiple of 128, take the split
 * product: per step a 128 x 128-tile MFMA product over up to four k slices (float32
 * partials), summed in slice order by the update that follows; 0 when the split does not
 * apply (the fused per-step kernel runs). No counterpart in the reference (its product is
 * one torch.matmul per step, rate/engine.py:157-300). */
int64_t wt_rate_split_bytes(const wt_rate_tables* tab, const wt_rate_operand* op, int64_t B);

/* wt_split_bf16 — hi = bf16(x), lo = bf16(x - hi), round to nearest even: x = hi + lo to
 * 2^-17 relative. The rate weight gradient's float32 product dL/dW = r^T dL/da
 * (rate/engine.py:367-376) is then taken as hi.hi + hi.lo + lo.hi on the bf16 matrix
 * cores (float32 accumulation and output), as accurate as the float32 product at 2.5x its
 * speed. No counterpart in the reference. n floats; x, hi, lo 16-byte aligned. */
int wt_split_bf16(const float* x, int64_t n, void* hi, void* lo, wt_stream_t stream);

/* wt_gemm_tn_split — C (M x N) = A^T B, or C += A^T B with accumulate != 0, for float32
 * A (K x M, row pitch lda), B (K x N, pitch ldb), C (pitch ldc), all row-major: the rate
 * networks' weight gradient sum over (trial, step) of rates x dL/da, a float32 product in
 * the reference (rate/engine.py:365-377). Each operand element is split in registers into
 * bf16 hi + lo (x = hi + lo to 2^-18) and the product taken as hi.hi + hi.lo + lo.hi on
 * the bf16 matrix cores with float32 accumulation: every term within 3 * 2^-18 of
 * |a_k b_k|. Deterministic. */
int wt_gemm_tn_split(const float* A, int64_t lda, const float* B, int64_t ldb, float* C,
                     int64_t ldc, int64_t K, int64_t M, int64_t N, int32_t accumulate,
                     wt_stream_t stream);

/* wt_edge_sources — edge_src[e] = the source of edge e (E = indptr[n_src]). */
int wt_edge_sources(const int64_t* indptr, int64_t n_src, int64_t* edge_src,
                    wt_stream_t stream);

/* wt_events_count / wt_events_fill — per source, the nonzero entries of an activity
 * (BT, n) f32 (spikes, or inputs), in ascending row (trial*T + step) order: the event
 * lists the weight gradients take. Replaces the torch nonzero / argsort / bincount that
 * form them around the reference's weight_gradient (network_simulators/engine.py:327-350).
 * count writes indptr (n+1) int64 (indptr[n] = number of events) and fills scratch
 * (wt_events_scratch_bytes: per 256-row chunk and source, the count and the nonzero rows
 * as bits); fill, with the same scratch, writes bt (indptr[n]) int32 and, unless value is
 * NULL (activity known to be 0 or 1: spikes; the rows then come from the bits, without a
 * second read of the activity), value (indptr[n]) f32.
 * BT = B*T rows (b*T + t); fill writes each event's row as b*T_pad + t (T_pad >= T: the
 * pitch of rows padded per trial; T_pad = T for the rows as they are). Deterministic. BT
 * may have at most 65535 * 256 rows. */
int64_t wt_events_scratch_bytes(int64_t BT, int64_t n);
int wt_events_count(const float* activity, int64_t BT, int64_t n, void* scratch,
                    int64_t* indptr, wt_stream_t stream);
int wt_events_fill(const float* activity, int64_t BT, int64_t n, const void* scratch,
                   const int64_t* indptr, int32_t* bt, float* value, int64_t T,
                   int64_t T_pad, wt_stream_t stream);

/* wt_gate_scan — a feedforward pathway's presynaptic dynamics stepped through a chunk,
 * replacing gate_scan (network_simulators/kernels.py:87-129; the step of
 * network_simulators/network.py:186-223). x (B, T, n_in) f32 the chunk's input; the
 * pathway's n source rows are input columns rows[0 .. n-1] (int64, each in [0, n_in));
 * params (5,) f32: saturation c, gating decay d, release probability at rest U, decays
 * d_D, d_F. gating (B, R) f32, updated in place: with stp_col >= 0 the release
 * probabilities u (columns stp_col ..) and resources (stp_col + n ..), with sat_col >= 0
 * the receptors' gating (sat_col ..); at least one of them. factors (B, T, n) f32: each
 * step's factor f (the pathway's input is x f). Every operation rounded as torch rounds
 * it on the CPU. */
int wt_gate_scan(const float* x, int64_t B, int64_t T, int64_t n_in, const int64_t* rows,
                 int64_t n, const float* params, float* gating, int64_t R, int64_t stp_col,
                 int64_t sat_col, float* factors, wt_stream_t stream);

/* wt_weight_gradient — dL/dW on the connectome's support (its edges), event-driven:
 * grad_w[e] = sum over the events i of src(e) of ev_val[i] * grad_A[k, ev_bt[i], tgt(e)]
 * with k = pathway_offset + pathway(src(e)). Events of source j are ev_indptr[j] ..
 * ev_indptr[j+1]-1; ev_bt = b*T + t ascending (int32), ev_val the presynaptic activity
 * there (NULL: 1 at every event, spikes).
 * Replaces: network_simulators/engine.py:327-350 weight_gradient (a dense GEMM over
 * every (source, target) pair, most of whose products are zero); the reference's
 * learnt projections multiply the gradient by a mask that is zero off the support
 * (projections.py:164, :216). grad_A (K,B,T,N); grad_w (E,) f32 overwritten. */
int wt_weight_gradient(const wt_side* side, const int64_t* edge_src, int64_t n_edges,
                       const int64_t* ev_indptr, const int32_t* ev_bt, const float* ev_val,
                       const float* grad_A, int64_t B, int64_t T, int64_t N,
                       int64_t pathway_offset, float* grad_w, wt_stream_t stream);

/* wt_filter_forward — the causal double-exponential filter of spike trains, replacing
 * _DoubleExponential.forward / _filter_forward (training_utils/filtering.py:75-86,103-123).
 * x, rise, smooth (B, T, N) f32 contiguous; carried_rise, carried_smooth (B, N) f32 or NULL
 * (zero). rise[t] = a_rise rise[t-1] + x[t], smooth[t] = a_decay smooth[t-1] + rise[t], the
 * carried state entering undecayed at t = 0; each multiply and add rounded separately.
 * B, N below 2^32, T below 2^32 - 8. */
int wt_filter_forward(const float* x, const float* carried_rise, const float* carried_smooth,
                      float* rise, float* smooth, float a_rise, float a_decay, int64_t B,
                      int64_t T, int64_t N, wt_stream_t stream);

/* wt_filter_backward — its reverse recursion, replacing _DoubleExponential.backward /
 * _filter_backward (training_utils/filtering.py:88-97,125-135): gs = g[t] + a_decay gs,
 * gr = gs + a_rise gr, grad_x[t] = gr, for t = T-1 .. 0. grad_smooth, grad_x (B, T, N) f32
 * contiguous. No gradient flows into the carried states or through rise. */
int wt_filter_backward(const float* grad_smooth, float* grad_x, float a_rise, float a_decay,
                       int64_t B, int64_t T, int64_t N, wt_stream_t stream);

/* wt_weight_gradient_by_target — the same sums (in a fixed order of their own: a
 * wave's 64 lanes over consecutive events, then a tree), grouped by (pathway, target)
 * row: grad_A (n_pathways, BT, N) is the side's dL/da, first transposed into rows
 * (n_pathways * N, BT) f32 (caller's scratch, overwritten), row k * N + n = dL/da_k over
 * b*T+t for target n; the incoming synapses of row kn are in_edge[in_indptr[kn] ..
 * in_indptr[kn+1]-1] (edge indices, each edge in the row of its source's pathway). One
 * workgroup per row reads it once into LDS. Every edge listed is overwritten; edges
 * listed in no row are left alone. With grad_A NULL, rows already holds the rows (row
 * length BT, e.g. B*T_pad from wt_cond_scan_backward's grad_A_rows, the events' rows in
 * that pitch) and nothing is transposed. Replaces: as wt_weight_gradient. */
int wt_weight_gradient_by_target(const int64_t* edge_src, int64_t n_edges,
                                 const int64_t* in_indptr, const int64_t* in_edge,
                                 int64_t n_pathways, int64_t N, const int64_t* ev_indptr,
                                 const int32_t* ev_bt, const float* ev_val,
                                 const float* grad_A, int64_t BT, float* rows, float* grad_w,
                                 wt_stream_t stream);

int wt_device_info(int64_t* n_cu, int64_t* max_lds_bytes);

#ifdef __cplusplus
}
#endif
#endif /* WIRETORCH_AMD_H */
