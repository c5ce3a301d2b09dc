/*
 * dsx.h -- C ABI of libdsx.so, the gfx950 (MI355X) ZeRO optimizer step.
 *
 * The step over one flat partition of n elements is three stream-ordered
 * launches with no host synchronisation between them:
 *
 *   K1 dsx_unscale_norm   16-bit grads -> per-block fp64 partial sums of
 *                         (g * inv_scale)^2; a non-finite grad makes the sum
 *                         non-finite, which is how overflow is detected.
 *   K0 dsx_finalize       partials -> global norm, found_inf, clip
 *                         coefficient, optimizer step t, fp32 step scalars,
 *                         and the loss-scaler update (device-resident state).
 *   K2 dsx_adamw_flat     one pass: unscale, clip, AdamW, 16-bit cast.
 *                         Reads 14 B/elt and writes 14 B/elt; returns at
 *                         once (no memory traffic) when K0 decided to skip.
 *   K3 dsx_*_multi        K1/K2 over a ragged list of tensors, driven by a
 *                         chunk table (one launch per pass for any count).
 *
 * The one-call steps (dsx_zero_step_flat, dsx_zero_step_plan,
 * dsx_zero_step_dev) run without a K0 launch where the fold's limits allow
 * (at most 512 partials, every nonempty group at least 4 elements), with the
 * same results: small partitions (dsx_set_tuning_fold) as K1 and K2 with
 * K0's finalize folded in, larger ones with it folded into the first of K2's
 * parts.
 *
 * Conventions
 *   - Every pointer argument is a DEVICE pointer owned by the caller, except
 *     where a comment says "host". The library allocates no device memory;
 *     scratch (the fp64 partials) is passed in by the caller.
 *   - Element counts are int64_t. Flat buffers must be 16-byte aligned; any n
 *     is accepted (the n % 8 tail is handled in-kernel).
 *   - Grads are DSX_F16, DSX_BF16 or DSX_F32 (fp32 training: the grad is
 *     read as is); param16 is DSX_F16 or DSX_BF16.
 *   - Work is enqueued on `stream` (a hipStream_t passed as void*; NULL means
 *     the null stream). No call synchronises the host with the device.
 *   - Return value: 0 on success; DSX_EINVAL (== hipErrorInvalidValue) for a
 *     rejected argument; otherwise the hipError_t of a failed launch.
 *     dsx_last_error() returns a thread-local message for the last failure.
 *
 * Arithmetic (fp32, in this order, no FMA contraction except where named;
 * the roundings of torch.optim.AdamW's default multi-tensor path on a GPU):
 *   g  = f32(g16) * inv_scale;  g = g * clip_coef
 *   p  = p * decay                               decay = f32(1 - lr*wd)
 *   m  = fma(w1, g - m, m)        if |w1| < .5, else fma(-(g - m), 1 - w1, g)
 *   v  = v * b2;  v = fma(val2, g * g, v)        val2 = f32(1 - beta2)
 *   d  = sqrt(v) / bc2s + eps                    IEEE sqrt and division
 *   p  = fma(nss, m / d, p)                      nss = f32(-lr / bc1[t])
 *   p16 = round_to_nearest_even(p)
 */
#ifndef DSX_H_
#define DSX_H_

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Version 2: DsxState's last 16 bytes (reserved in version 1) hold the
 * one-shot clip and the step's entry values, which K0, K1 and the folded
 * K2/K3 read. */
#define DSX_ABI_VERSION 2

/* element types */
#define DSX_F32  0
#define DSX_F16  1
#define DSX_BF16 2

/* loss-scaler modes */
#define DSX_SCALE_NONE    0 /* bf16 / fp32: scale stays 1, overflow still skips */
#define DSX_SCALE_STATIC  1 /* fp16.loss_scale > 0 */
#define DSX_SCALE_DYNAMIC 2 /* fp16.loss_scale == 0 */

/* status codes */
#define DSX_OK     0
#define DSX_EINVAL 1

/* state error bits (DsxState.error) */
#define DSX_STATE_ERR_BC_TABLE 1 /* bias-correction table shorter than t */
#define DSX_STATE_ERR_GROUPS   2 /* device-side group inputs out of range */

/* upper bound on the partials one K1 launch may write */
#define DSX_MAX_PARTIALS 8192

/* upper bound on the parameter groups of one dsx_finalize_groups call */
#define DSX_MAX_GROUPS 16

/* The library's own scratch per GPU (dsx_zero_step_flat_noalloc): room for
 * DSX_NOALLOC_MAX_PARTIALS fp64 partials followed by one DsxStepScalars. */
#define DSX_NOALLOC_MAX_PARTIALS 8192
#define DSX_NOALLOC_SCRATCH_BYTES (8 * DSX_NOALLOC_MAX_PARTIALS + 256)

/* Device-resident optimizer + loss-scaler state (64 bytes). Write it with
 * dsx_state_init, or copy back one the library wrote (a checkpoint). A
 * caller that fills one itself must zero clip_once_coef, clip_once,
 * step_scale and step_t2: a nonzero clip_once arms a one-shot clip for the
 * next finalize. */
typedef struct DsxState {
  float   scale;          /* loss scale the next backward multiplies by      */
  int32_t good_steps;     /* clean steps since the last overflow or growth   */
  int32_t hyst_left;      /* overflows still tolerated before a backoff      */
  int32_t t;              /* AdamW step count; skipped steps do not count    */
  int64_t iter;           /* finalize calls so far                           */
  int64_t overflow_count; /* skipped steps so far                            */
  int32_t error;          /* DSX_STATE_ERR_* bits, sticky                    */
  int32_t last_skip;      /* 1 if the last finalize skipped                  */
  double  last_norm;      /* global grad norm seen by the last finalize      */
  float   clip_once_coef; /* clip coefficient armed by dsx_clip_prepare      */
  int32_t clip_once;      /* 1: the next finalize applies clip_once_coef     */
  float   step_scale;     /* scale as the last step began                    */
  int32_t step_t2;        /* 2 t + clip_once as the last step began          */
} DsxState;

/* Loss-scaler configuration (by value). */
typedef struct DsxScalerConfig {
  int32_t mode;           /* DSX_SCALE_*                                     */
  int32_t window;         /* loss_scale_window: clean steps per growth       */
  int32_t hysteresis;     /* overflows tolerated before a backoff (>= 1)     */
  int32_t reserved;
  float   min_scale;      /* min_loss_scale                                  */
  float   growth_factor;  /* 2.0                                             */
  float   backoff_factor; /* 0.5                                             */
  float   reserved2;
} DsxScalerConfig;

/* AdamW hyper-parameters for one step (by value; host doubles, as torch). */
typedef struct DsxAdamwHyper {
  double lr;
  double beta1;
  double beta2;
  double eps;
  double weight_decay;
  double max_grad_norm;   /* <= 0 disables clipping                          */
  double clip_eps;        /* added to the norm in the clip coefficient (1e-6) */
} DsxAdamwHyper;

/* fp32 scalars of one step, written by dsx_finalize (64 bytes). */
typedef struct DsxStepScalars {
  int32_t skip;           /* nonzero: overflow (or error), K2 does nothing   */
  int32_t t;              /* step number used for bias correction            */
  float   inv_scale;      /* 1 / scale used by this step's backward          */
  float   clip_coef;      /* 1.0f when not clipping                          */
  float   decay;          /* f32(1 - lr*wd), 1.0f when wd == 0               */
  float   w1;             /* f32(1 - beta1), lerp weight                     */
  float   w1c;            /* 1.0f - w1                                       */
  float   b2;             /* f32(beta2)                                      */
  float   val2;           /* f32(1 - beta2)                                  */
  float   eps;            /* f32(eps)                                        */
  float   bc2s;           /* f32(sqrt(1 - beta2^t))                          */
  float   nss;            /* f32(-(lr / (1 - beta1^t)))                      */
  double  sumsq;          /* sum of squared unscaled grads (fp64)            */
  double  norm;           /* sqrt(sumsq)                                     */
} DsxStepScalars;

/* One tensor of a ragged list (K3). master/exp_avg/exp_avg_sq fp32;
 * grad of the call's grad dtype; param16 (16-bit, may be NULL: no cast
 * written) of the call's param dtype. `group` selects scalars[group]. */
typedef struct DsxTensorRef {
  float*      master;
  float*      exp_avg;
  float*      exp_avg_sq;
  void*       param16;
  const void* grad;
  int64_t     numel;
  int32_t     group;
  int32_t     reserved;
} DsxTensorRef;

/* One chunk of a ragged list: elements [start, start+len) of tensor `tensor`.
 * The kernels take both tables as given (they live in device memory, out of
 * the host's sight): each chunk needs 0 <= tensor < the tensor count,
 * start >= 0, len >= 0 and start + len <= that tensor's numel, and each
 * tensor's arrays numel elements; dsx_build_chunks writes such tables. The
 * tables are read through the scalar (constant) cache, so they must not
 * change while a launch that reads them runs. */
typedef struct DsxChunk {
  int32_t tensor;
  int32_t reserved;
  int64_t start;
  int64_t len;
} DsxChunk;

/* ---- library ---------------------------------------------------------- */

int         dsx_abi_version(void);
const char* dsx_last_error(void);

/* Launch-shape override for the current process (library tuning; no
 * counterpart in the reference): K1 blocks per CU (default 2), K2 blocks per
 * CU (0, the default, picks by n: below 3 * 2^27 elements one trip per block
 * while that takes at most 32 blocks per CU, else one block per CU), K2
 * slots per thread per trip (2, 4 or 8; 0, the default, picks 2 below
 * 3 * 2^27 elements and 4 from there on) and the nontemporal hint (0/1). */
int dsx_set_tuning(int k1_blocks_per_cu, int k2_blocks_per_cu, int k2_unroll,
                   int nontemporal);

/* K2's grid and pacing: k2_blocks_per_cu blocks on k2_cu_eighths eighths of
 * the CUs (1..8; 0, the default, picks 7 for n >= 3 * 2^27 elements and 8
 * below), and whether each wave waits for its stores to complete before the
 * next trip's loads (drain 0/1; -1, the default, drains from 3 * 2^27
 * elements on). On MI355X a large partition's 50:50 read/write stream runs
 * faster with fewer requests in flight. No counterpart in the reference. */
int dsx_set_tuning_k2(int k2_cu_eighths, int drain);

/* K2 over a partition of more than chunk_elems elements runs as consecutive
 * launches of at most about chunk_elems elements (equal parts, multiples of
 * 1024 elements), each with the launch shape of its own size; 0 runs one
 * launch. Default 2^26: on MI355X one launch over a large partition loses
 * bandwidth as the partition grows, while 64 Mi-element launches hold the
 * mid-size rate. Applies to dsx_adamw_flat, dsx_zero_step_flat and
 * dsx_traffic_probe_flat. chunk_elems must be 0 or >= 2^20. No counterpart
 * in the reference. */
int dsx_set_tuning_k2_chunk(int64_t chunk_elems);

/* One-call steps (dsx_zero_step_flat, dsx_zero_step_plan and the no-
 * allocation variant) over at most max_elems elements, with at most 512
 * partials and every nonempty group at least 4 elements, run as two
 * launches: K1, which also records the entry scale, t and one-shot clip flag
 * in the state's step_scale / step_t2, and K2 with K0's finalize folded in
 * (every K2 block reduces the partials and decides the step itself, with
 * K0's code and order, so the bits are K0's; one extra block writes the
 * state and the step records). The folded K2 takes K2's one-trip grid (2
 * slots per thread, at most 32 blocks per CU) whatever dsx_set_tuning and
 * dsx_set_tuning_k2 set. Above max_elems (same limits), K0's finalize is
 * folded into the first of K2's parts alone, launched one block per CU, and
 * the other parts read the records it writes. 0 always runs K1, K0, K2.
 * Default 3 * 2^23 (one and a half sweeps of K2's one-trip grid on 256 CUs).
 * No counterpart in the reference. */
int dsx_set_tuning_fold(int64_t max_elems);

/* The same for K3 (dsx_adamw_multi): blocks per CU (the grid is also capped
 * at the chunk count; 0, the default, picks the shape from the chunk count,
 * always with 2 slots: one chunk per block up to 20 chunks per CU, one block
 * per CU below 256 chunks per CU, about four chunks per block with the drain
 * from there on), slots per thread per
 * trip (1, 2 or 4; used when blocks per CU is set), the nontemporal hint and
 * K2's per-trip drain (0/1; -1, the default, as the shape decides). No
 * counterpart in the reference. */
int dsx_set_tuning_multi(int k3_blocks_per_cu, int k3_unroll, int nontemporal,
                         int drain);

/* Partials a K1 launch over n elements should use on the current device
 * (a multiple of the CU count, <= DSX_MAX_PARTIALS). */
int32_t dsx_suggest_partials(int64_t n);

/* Number of chunks dsx_build_chunks produces (host only, no GPU). */
int64_t dsx_count_chunks(const int64_t* numels /* host */, int32_t ntensors,
                         int64_t chunk_elems);

/* Fill `out` (host, capacity cap) with the chunk table of a ragged list.
 * Returns the count, or -1 (with dsx_last_error) on bad arguments. */
int64_t dsx_build_chunks(const int64_t* numels /* host */, int32_t ntensors,
                         int64_t chunk_elems, DsxChunk* out /* host */,
                         int64_t cap);

/* ---- state ------------------------------------------------------------ */

/* Write an initial DsxState (scale, hysteresis; counters zero) on `stream`.
 * Replaces GradScaler(init_scale=2**initial_scale_power, ...) construction,
 * Src/zero/optimizer.py:102-110; fields Src/zero/__init__.py:103-109. */
int dsx_state_init(DsxState* state, float init_scale, int32_t hysteresis,
                   void* stream);

/* ---- K1: unscale + inf/NaN detect + squared L2 norm ------------------- */

/* partials[0..nparts) = per-block sums of (f32(g) * inv_scale)^2 in fp64,
 * inv_scale = f32(1 / (double)state->scale). Grads are only read.
 * Replaces Src/zero/utils.py:126-154 (compute_norm, one .item() per
 * tensor) and the unscale/found_inf of GradScaler the engine intends
 * (Src/zero/optimizer.py:236-242, 276-298). */
int dsx_unscale_norm(const void* grad, int grad_dtype, int64_t n,
                     const DsxState* state, double* partials, int32_t nparts,
                     void* stream);

/* K1 folded into a copy: dst[0..n) = src[0..n) (grad dtype, both 16-byte
 * aligned, not overlapping) and partials[0..nparts) = per-block sums of
 * (f32(src) * inv_scale)^2 in fp64, as dsx_unscale_norm sums them. This is
 * the copy the flat form's post-accumulate hook makes of the grad autograd
 * produced (replacing the `param.grad` copy of the reference's packing,
 * Src/zero/stage1.py:137-144, Src/zero/stage2.py:210-218), with the norm of
 * Src/zero/utils.py:126-154 taken on the way. */
int dsx_copy_unscale_norm(const void* src, void* dst, int grad_dtype, int64_t n,
                          const DsxState* state, double* partials,
                          int32_t nparts, void* stream);

/* out[b] = sum of partials[offsets[b] .. offsets[b+1]) for b < nseg, each in
 * a fixed order (offsets: nseg + 1 nondecreasing DEVICE int64 indices into
 * partials): one partial per parameter from the block partials of its
 * dsx_copy_unscale_norm, for K0. No counterpart in the reference. */
int dsx_reduce_segments(const double* partials, const int64_t* offsets,
                        int32_t nseg, double* out, void* stream);

/* ---- clip_grad_norm_: norms of any type, one-shot clip ---------------- */

/* partials[0..nparts) = per-block fp64 partials of the norm of type
 * norm_type over x = f32(g) * inv_scale (inv_scale as dsx_unscale_norm):
 * sums of x^2 (norm_type 2), of |x| (1), of |x|^norm_type (any other finite
 * norm_type > 0, pow in fp64), or maxima of |x| (norm_type = +inf; NaN if
 * any x is NaN). norm_type must be > 0 (finite or +inf). Replaces
 * compute_norm, Src/zero/utils.py:126-154 (inf: :141-143, p: :146-152), and
 * the stages' p-norms, Src/zero/stage1.py:596-600, Src/zero/stage2.py:690-695. */
int dsx_norm_partials(const void* grad, int grad_dtype, int64_t n,
                      const DsxState* state, double norm_type, double* partials,
                      int32_t nparts, void* stream);

/* The same over the chunks of a tensor list. */
int dsx_norm_partials_multi(const DsxTensorRef* tensors, const DsxChunk* chunks,
                            int64_t nchunks, int grad_dtype,
                            const DsxState* state, double norm_type,
                            double* partials, int32_t nparts, void* stream);

/* One block: the norm of type norm_type from dsx_norm_partials' partials
 * (sqrt of the sum for 2, sum^(1/p) for other finite p, the sum for 1, the
 * maximum for inf) into *norm_out (device double), and arms state's one-shot
 * clip: the next finalize multiplies the grads by max_norm / (norm +
 * clip_eps) (rounded to fp32; 1 unless norm > max_norm) instead of applying
 * the configured max_grad_norm, whether that step is applied or skipped,
 * and disarms it. max_norm >= 0. Replaces the in-place clip of
 * clip_grad_norm_, Src/zero/optimizer.py:324-341 -> Src/zero/utils.py:187-216,
 * Src/zero/stage1.py:549-582, Src/zero/stage2.py:683-725. */
int dsx_clip_prepare(const double* partials, int32_t nparts, double norm_type,
                     double max_norm, double clip_eps, DsxState* state,
                     double* norm_out, void* stream);

/* ---- K0: finalize ------------------------------------------------------ */

/* Reduce the partials; decide skip (non-finite sum); on a clean step advance
 * t and emit the step scalars (clip coefficient max_norm/(norm+clip_eps) if
 * norm > max_norm, or the one dsx_clip_prepare armed); update the loss
 * scaler. bc_table holds bc_len pairs
 * {1 - beta1^t, (1 - beta2^t)^0.5} for t = 1..bc_len, computed on the host
 * in double exactly as torch/optim/adam.py:529-535 does.
 * Replaces Src/zero/optimizer.py:212-274 (skip/clip/update order),
 * Src/zero/utils.py:187-216 (clip) and GradScaler.update
 * (Src/zero/optimizer.py:265-266). */
int dsx_finalize(const double* partials, int32_t nparts, DsxState* state,
                 DsxScalerConfig scaler, DsxAdamwHyper hyper,
                 const double* bc_table, int32_t bc_len, DsxStepScalars* out,
                 void* stream);

/* The same for up to DSX_MAX_GROUPS parameter groups (torch param_groups
 * with their own lr / betas / eps / weight_decay): one skip decision, norm,
 * clip coefficient (from hypers[0].max_grad_norm) and scaler update; out[g]
 * receives group g's scalars. hypers, bc_tables and t_offsets are HOST
 * arrays of ngroups entries (bc_tables[g] is a device table as above; the
 * tables share bc_len); group g steps with t - t_offsets[g] (a group added
 * after k steps starts its own count at 1, as torch's per-parameter step
 * does). Replaces the per-group loop of torch.optim.AdamW.step. */
int dsx_finalize_groups(const double* partials, int32_t nparts, DsxState* state,
                        DsxScalerConfig scaler, const DsxAdamwHyper* hypers,
                        const double* const* bc_tables,
                        const int32_t* t_offsets, int32_t ngroups,
                        int32_t bc_len, DsxStepScalars* out, void* stream);

/* Per-step inputs of dsx_finalize_dev, held in DEVICE memory so that a
 * captured graph reads the current values at every replay (1112 bytes). */
typedef struct DsxGroupsDev {
  DsxAdamwHyper  hyper[DSX_MAX_GROUPS];
  const double*  bc_table[DSX_MAX_GROUPS];  /* device tables, as dsx_finalize */
  int32_t        t_offset[DSX_MAX_GROUPS];
  int32_t        ngroups;
  int32_t        bc_len;
  int64_t        reserved[2];
} DsxGroupsDev;

/* dsx_finalize_groups with its per-group inputs read from `groups` (device
 * memory) instead of kernel arguments: the form to capture in a HIP graph
 * (the host updates `groups` with an async copy before each replay). `out`
 * has room for max_groups scalars and all of them are written: slots at or
 * past groups->ngroups get skip = 1. A groups->ngroups outside
 * [1, max_groups] or an invalid hyper-parameter sets DSX_STATE_ERR_GROUPS and
 * skips the step (every slot). No counterpart in the reference (it has no
 * graph path). */
int dsx_finalize_dev(const double* partials, int32_t nparts, DsxState* state,
                     DsxScalerConfig scaler, const DsxGroupsDev* groups,
                     int32_t max_groups, DsxStepScalars* out, void* stream);

/* Copies the HOST block `groups` into the device block `dst` in stream
 * order (a one-wave kernel that takes the block as its argument: no host
 * staging buffer, no DMA copy, nothing to wait for on the host). Checks the
 * block as dsx_finalize_groups checks its arrays. Used before each replay of
 * a graph that holds dsx_finalize_dev. No counterpart in the reference. */
int dsx_groups_upload(const DsxGroupsDev* groups, DsxGroupsDev* dst,
                      void* stream);

/* ---- K2: AdamW + cast over a flat partition -------------------------- */

/* In place on master/exp_avg/exp_avg_sq (fp32, n elements); writes param16
 * (param_dtype F16/BF16; may be NULL). No-op when scalars->skip.
 * Replaces torch.optim.AdamW.step called at Src/zero/stage1.py:522-525 and
 * Src/zero/stage2.py:609-612, and FusedKernels.fused_adam_step,
 * Src/engine.py:871-890. */
int dsx_adamw_flat(float* master, float* exp_avg, float* exp_avg_sq,
                   void* param16, int param_dtype, const void* grad,
                   int grad_dtype, int64_t n, const DsxStepScalars* scalars,
                   void* stream);

/* Measurement only, no counterpart in the reference: K2's exact traffic
 * (grad, master, exp_avg and exp_avg_sq read; master, exp_avg, exp_avg_sq
 * and param16 written: 28 B per element) in K2's launch shape for n, with
 * the AdamW math left out. Writes back the values it reads and param16 =
 * RNE(master), so on a partition whose param16 is the cast of its master it
 * changes nothing. dtype is the grad and param16 type (F16 or BF16);
 * param16 is required. Timing it beside dsx_adamw_flat tells how close K2
 * runs to the ceiling of its own access pattern. */
int dsx_traffic_probe_flat(float* master, float* exp_avg, float* exp_avg_sq,
                           void* param16, int dtype, const void* grad,
                           int64_t n, void* stream);

/* K1 -> K0 -> K2 over one flat partition: the whole engine.step() of
 * Src/zero/optimizer.py:212-274 for stage 1/2 at world size 1. `partials`
 * has room for nparts doubles; `out` receives this step's scalars. */
int dsx_zero_step_flat(float* master, float* exp_avg, float* exp_avg_sq,
                       void* param16, int param_dtype, const void* grad,
                       int grad_dtype, int64_t n, DsxState* state,
                       DsxScalerConfig scaler, DsxAdamwHyper hyper,
                       const double* bc_table, int32_t bc_len,
                       double* partials, int32_t nparts, DsxStepScalars* out,
                       void* stream);

/* What a flat partition's step needs that stays fixed from step to step
 * (the drop-in optimizer builds it once). Parameter group g covers elements
 * [group_end[g-1], group_end[g]) (group_end[-1] = 0): every boundary but the
 * last a multiple of 8 elements, the last equal to n. */
typedef struct DsxFlatPlan {
  float*          master;
  float*          exp_avg;
  float*          exp_avg_sq;
  void*           param16;      /* may be NULL                              */
  const void*     grad;
  int64_t         n;
  int32_t         param_dtype;
  int32_t         grad_dtype;
  DsxState*       state;
  double*         partials;     /* nparts doubles                           */
  DsxStepScalars* out;          /* ngroups entries                          */
  int32_t         nparts;
  int32_t         ngroups;
  DsxScalerConfig scaler;
  int64_t         group_end[DSX_MAX_GROUPS];
} DsxFlatPlan;

/* K1 -> K0 -> K2 (one K2 call per non-empty group range) in one call: the
 * whole step of the flat drop-in optimizer with parameter groups. plan and
 * groups are HOST structs (groups holds this step's hyper-parameters, bias
 * tables and t offsets, as dsx_finalize_groups takes them); both are checked
 * at every call. Replaces ZeROOptimizer.step, Src/zero/optimizer.py:212-274,
 * with torch AdamW's per-group loop behind Src/zero/stage2.py:609-612. */
int dsx_zero_step_plan(const DsxFlatPlan* plan /* host */,
                       const DsxGroupsDev* groups /* host */, void* stream);

/* dsx_zero_step_plan with the group block in DEVICE memory (written, e.g.,
 * by dsx_groups_upload), read by the kernels when they run: the launches
 * can be recorded into a HIP graph once and replayed, with a new block
 * uploaded between replays. The block is checked on the device (as
 * dsx_finalize_dev checks it: a bad block skips the step and sets
 * DSX_STATE_ERR_GROUPS); records are written for plan->ngroups slots. The
 * same kernels and bits as dsx_zero_step_plan (two launches where
 * dsx_set_tuning_fold's bound allows, else three). No counterpart in the
 * reference (it has no graph path). */
int dsx_zero_step_dev(const DsxFlatPlan* plan /* host */,
                      const DsxGroupsDev* groups_dev, void* stream);

/* dsx_zero_step_flat that allocates nothing and takes no scratch buffer:
 * K1's partials and (when out is NULL) K0's step scalars live in a static
 * device array of the library, DSX_NOALLOC_SCRATCH_BYTES per GPU, held until
 * the process ends. No counterpart in the reference; it is for callers that
 * cannot allocate device memory (code recorded into a HIP graph, tight
 * serving loops, harnesses that forbid hipMalloc). The caller still passes
 * the inputs and outputs (the flat buffers, state, bc_table; out may be NULL).
 * nparts: 0 picks dsx_suggest_partials(n); above DSX_NOALLOC_MAX_PARTIALS is
 * rejected with DSX_EINVAL. `stream` must belong to the current device. The
 * first call on each device resolves the array's address
 * (hipGetSymbolAddress), so make it outside stream capture. Calls share their
 * GPU's array: calls that overlap on one GPU (different streams, or host
 * threads without ordering) race. Results are bit-identical to
 * dsx_zero_step_flat with the same nparts. */
int dsx_zero_step_flat_noalloc(float* master, float* exp_avg,
                               float* exp_avg_sq, void* param16,
                               int param_dtype, const void* grad,
                               int grad_dtype, int64_t n, DsxState* state,
                               DsxScalerConfig scaler, DsxAdamwHyper hyper,
                               const double* bc_table, int32_t bc_len,
                               int32_t nparts, DsxStepScalars* out,
                               void* stream);

/* ---- K3: ragged lists (multi-tensor apply) ---------------------------- */

/* K1 over the chunks of a tensor list (tensors/chunks are device arrays).
 * Replaces the per-tensor loop of Src/zero/utils.py:147-152. */
int dsx_unscale_norm_multi(const DsxTensorRef* tensors, const DsxChunk* chunks,
                           int64_t nchunks, int grad_dtype,
                           const DsxState* state, double* partials,
                           int32_t nparts, void* stream);

/* K2 over the chunks of a tensor list; per element identical to
 * dsx_adamw_flat. Replaces torch AdamW's per-tensor loop
 * (torch/optim/adam.py:396) behind Src/zero/stage2.py:609-612. */
int dsx_adamw_multi(const DsxTensorRef* tensors, const DsxChunk* chunks,
                    int64_t nchunks, int param_dtype, int grad_dtype,
                    const DsxStepScalars* scalars, void* stream);

/* The ragged list's whole step in one call: K1 over the list, K0 with the
 * HOST group block `groups` (as dsx_finalize_groups takes it; checked here),
 * K3 -- or, for lists of at most dsx_set_tuning_fold's bound in elements
 * (numel, the sum of the chunk lengths) with at most 512 partials and at
 * most 20 chunks per CU, two launches: K1 recording the entry values, and K3
 * with K0's finalize folded in (every block decides the step with K0's code;
 * one extra block writes the state and the records), the same bits. out
 * holds groups->ngroups records. Replaces ZeROOptimizer.step over a list of
 * tensors (Src/zero/optimizer.py:212-274, torch AdamW's per-tensor loop
 * behind Src/zero/stage2.py:609-612). */
int dsx_zero_step_multi(const DsxTensorRef* tensors, const DsxChunk* chunks,
                        int64_t nchunks, int64_t numel, int param_dtype,
                        int grad_dtype, DsxState* state, DsxScalerConfig scaler,
                        const DsxGroupsDev* groups /* host */, double* partials,
                        int32_t nparts, DsxStepScalars* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSX_H_ */
