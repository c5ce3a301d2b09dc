// dsx_step.hip -- gfx950 kernels and C ABI of libdsx.so (see include/dsx.h).
//
// The ZeRO optimizer step over one flat partition, as the reference's
// ZeROOptimizer.step (Src/zero/optimizer.py:212-274) orders it: overflow
// check / skip -> unscale -> norm -> clip -> AdamW -> loss-scaler update,
// with the AdamW arithmetic of torch.optim.AdamW (torch/optim/adam.py:347-552)
// that the reference calls at Src/zero/stage1.py:522-525 and
// Src/zero/stage2.py:609-612.
//
// Everything is HBM-bound streaming. K2 moves 28 B per element with 16-bit
// grads (grad 2 + master/m/v 12 read, master/m/v 12 + param16 2 written) and
// K1 2 B per element. The kernels are grid-stride loops over 4-element slots
// (fp32 in 16-byte loads, 16-bit values in 8-byte loads) so that every load
// and store instruction of a wave touches one contiguous span; several slots
// per thread are loaded before any is used, to keep bytes in flight.
//
// Compile with -ffp-contract=off: the element math must round exactly where
// torch rounds, and the only fused multiply-adds are the explicit fmaf calls
// that mirror the fused operations of torch's GPU kernels (lerp, addcmul,
// addcdiv).

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>
#include <string.h>
#include <math.h>

#include <mutex>
#include <type_traits>

#include "dsx.h"

static_assert(sizeof(DsxState) == 64, "DsxState layout");
static_assert(sizeof(DsxScalerConfig) == 32, "DsxScalerConfig layout");
static_assert(sizeof(DsxAdamwHyper) == 56, "DsxAdamwHyper layout");
static_assert(sizeof(DsxStepScalars) == 64, "DsxStepScalars layout");
static_assert(sizeof(DsxTensorRef) == 56, "DsxTensorRef layout");
static_assert(sizeof(DsxChunk) == 24, "DsxChunk layout");
static_assert(sizeof(DsxGroupsDev) == 1112, "DsxGroupsDev layout");
static_assert(sizeof(DsxFlatPlan) == 248, "DsxFlatPlan layout");

// Scratch of dsx_zero_step_flat_noalloc: K1's fp64 partials, then K0's step
// scalars. One copy per GPU, held until the process ends. Host code never
// uses this name as an address (on the host it is a stand-in, not device
// memory): it passes the pointer hipGetSymbolAddress returns for the current
// device (noalloc_scratch below).
constexpr size_t kScratchScalarsOffset = sizeof(double) * DSX_NOALLOC_MAX_PARTIALS;
static_assert(kScratchScalarsOffset % 256 == 0, "step scalars start 256-byte aligned");
static_assert(kScratchScalarsOffset + sizeof(DsxStepScalars) <= DSX_NOALLOC_SCRATCH_BYTES, "scratch layout");
static __device__ __align__(256) unsigned char scratch[DSX_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;

typedef float    f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

thread_local char g_err[512];

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail((int)e, "%s: launch failed: %s", what, hipGetErrorString(e));
  return DSX_OK;
}

__host__ __device__ inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool is16(int dt) { return dt == DSX_F16 || dt == DSX_BF16; }
bool is_grad_dtype(int dt) { return dt == DSX_F16 || dt == DSX_BF16 || dt == DSX_F32; }

// ---- launch shape ----------------------------------------------------------

// Defaults from launch-shape sweeps of the library's kernels on MI355X over
// partitions of 1.0e6 to 1.0e9 elements. K2 (256-thread blocks) has three
// regimes. Up to 32 blocks per CU of one trip each (2 slots per thread: up to
// 16.8e6 elements), every block makes one trip, so that all loads are in
// flight at once (2-12% faster than one block per CU from 2 Mi to 16 Mi
// elements; the same at 1 Mi and 32 Mi). Up to ~2.5e8 elements, one block per
// CU with 2 slots per thread per trip is best. From ~5e8 elements up,
// K2's 50:50 read/write stream runs best when the chip issues fewer requests
// than it could: 4 slots per thread, each wave waiting for its own stores to
// complete before it loads the next trip ("drain"), and blocks on only 7 of
// every 8 CUs (1.0e9 elements: 5.12 ms against 5.19 on every CU and 5.24 in
// the small-partition shape; 5e8: 2.51 against 2.55 ms). K1 (read-only) runs
// best with two blocks per CU. Nontemporal hints help both by a few percent.
constexpr int64_t kK2LargeN = int64_t(3) << 27;  // K2's large-partition shape from here on
constexpr int64_t kMaxGridBlocks = int64_t(1) << 22;  // 2^30 work-items of kBlock threads
constexpr int64_t kK2OneTripPerCu = 32;  // K2's one-trip grid up to this many blocks per CU
constexpr int64_t kK3OneChunkPerCu = 20;  // K3: one chunk per block up to this many chunks per CU

struct Tuning {
  int k1_blocks_per_cu = 2;
  // K2's shape; 0 (-1 for the drain) picks by n: below kK2LargeN 2 slots,
  // no drain, and one trip per block while that takes at most
  // kK2OneTripPerCu blocks per CU, else one block per CU on 8 eighths; from
  // kK2LargeN on one block per CU on 7 eighths, 4 slots, drain.
  int k2_blocks_per_cu = 0;
  int k2_cu_eighths = 0;  // blocks on this many eighths of the CUs
  int k2_unroll = 0;      // slots per thread per trip: 2, 4 or 8
  int k2_drain = -1;      // wait for a trip's stores before the next trip's loads
  int nontemporal = 1;    // nontemporal hint on the streaming loads/stores
  int k3_blocks_per_cu = 0;  // 0: chosen per launch from the chunk count
  int k3_unroll = 1;         // slots per thread per trip in K3: 1, 2 or 4 (when not chosen)
  int k3_nontemporal = 1;
  int k3_drain = -1;         // the K2 drain in K3's slot loop (-1: as the default shape decides)
  // K2 over a partition above this many elements runs as consecutive
  // launches of about this many (0: one launch). One launch over a large
  // partition loses bandwidth as it grows (1.0e9 elements: 5.52 TB/s, 4.3e9:
  // 5.36); launches of 32-64 Mi elements in the mid-size shape hold 5.9-6.0
  // TB/s from 64 Mi to 4 Gi elements (16 Mi parts lose to launch gaps, 256 Mi
  // parts lose the gain; splitting below 64 Mi gains nothing).
  int64_t k2_chunk_elems = int64_t(1) << 26;
  // Steps over at most this many elements (with at most kFoldMaxParts
  // partials) run as two launches, K1 and K2 with the finalize folded in
  // (k2_adamw_fold), instead of K1, K0, K2; 0: always three launches.
  // 3 * 2^23: K2's one-trip grid on 256 CUs covers 2^24 elements, and up to
  // one and a half sweeps of it the fold still wins (eager flat step on
  // MI355X: 20 Mi elements 108.0 against 113.4 us, 24 Mi 130.7 against
  // 133.9; 32 Mi even, 48 Mi 267.9 against 256.2: every block also reduces
  // the partials).
  int64_t fold_max_elems = int64_t(3) << 23;
};
Tuning g_tune;

int cu_count() {
  static int cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64 && cache[dev] > 0) return cache[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  if (dev < 64) cache[dev] = cus;
  return cus;
}

// b > 0; exact for any a, with no intermediate that can overflow.
int64_t ceil_div(int64_t a, int64_t b) { return a / b + (a % b > 0 ? 1 : 0); }

// ---- element helpers -------------------------------------------------------

template <bool NT, typename T>
__device__ __forceinline__ T ld(const T* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <bool NT, typename T>
__device__ __forceinline__ void st(T* p, T v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// 16-bit storage value (low half of h) -> fp32; exact for both formats.
template <int DT>
__device__ __forceinline__ float h2f(uint32_t h) {
  if constexpr (DT == DSX_BF16) {
    return __uint_as_float(h << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
  }
}

// fp32 -> 16-bit, round to nearest even. NaN becomes the quiet NaN
// 0x7FC0 (bf16, as c10::BFloat16 does) or sign|0x7E00 (fp16).
template <int DT>
__device__ __forceinline__ uint32_t f2h(float x) {
  const uint32_t u = __float_as_uint(x);
  if constexpr (DT == DSX_BF16) {
    if (x != x) return 0x7FC0u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  } else {
    if (x != x) return ((u >> 16) & 0x8000u) | 0x7E00u;
    return (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)x);
  }
}

// Grad formats: element storage, the 4-element slot K2 loads, and how a
// 16-byte K1 slot unpacks.
template <int GD>
struct Grad {  // DSX_F16 / DSX_BF16
  using elem = uint16_t;
  using slot4 = u2;
  static constexpr int per16 = 8;
  __device__ static float one(elem e) { return h2f<GD>(e); }
  __device__ static void four(const slot4& s, float (&g)[4]) {
    g[0] = h2f<GD>(s.x); g[1] = h2f<GD>(s.x >> 16); g[2] = h2f<GD>(s.y); g[3] = h2f<GD>(s.y >> 16);
  }
  __device__ static double sumsq16(const u4& s, float inv, double acc) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float a = h2f<GD>(s[k]) * inv;
      const float b = h2f<GD>(s[k] >> 16) * inv;
      acc = __builtin_fma((double)a, (double)a, acc);
      acc = __builtin_fma((double)b, (double)b, acc);
    }
    return acc;
  }
};

template <>
struct Grad<DSX_F32> {
  using elem = float;
  using slot4 = f4;
  static constexpr int per16 = 4;
  __device__ static float one(elem e) { return e; }
  __device__ static void four(const slot4& s, float (&g)[4]) {
    g[0] = s[0]; g[1] = s[1]; g[2] = s[2]; g[3] = s[3];
  }
  __device__ static double sumsq16(const u4& s, float inv, double acc) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float a = __uint_as_float(s[k]) * inv;
      acc = __builtin_fma((double)a, (double)a, acc);
    }
    return acc;
  }
};

// Step scalars held in registers.
struct Sc {
  float inv, coef, decay, w1, w1c, b2, val2, eps, bc2s, nss;
  bool small;
};

__device__ __forceinline__ Sc load_sc(const DsxStepScalars& s) {
  Sc r;
  r.inv = s.inv_scale; r.coef = s.clip_coef; r.decay = s.decay;
  r.w1 = s.w1; r.w1c = s.w1c; r.b2 = s.b2; r.val2 = s.val2;
  r.eps = s.eps; r.bc2s = s.bc2s; r.nss = s.nss;
  r.small = fabsf(s.w1) < 0.5f;
  return r;
}

// One element of the step. Order and rounding are those of torch.optim.AdamW
// on a GPU -- its default multi-tensor path, torch/optim/adam.py:692-800,
// which the reference's stages reach through optimizer.step() -- measured
// bit for bit against torch on MI355X: unscale and clip are fp32 multiplies;
// _foreach_mul_(params, 1 - lr*wd); _foreach_lerp_ with a scalar weight is
// fma(w, end - self, self), or for |w| >= 0.5 end - (end - self) * (1 - w)
// as fma(-(end - self), 1 - w, end) (which keeps the sign of a zero as torch);
// _foreach_mul_(v, b2) then _foreach_addcmul_(v, g, g, 1 - b2) is
// fma(1 - b2, g * g, v); denom = sqrt(v) / bc2s + eps with IEEE sqrt and
// true division (_foreach_div_ by a list of scalars); _foreach_addcdiv_ is
// fma(value, m / denom, p).
__device__ __forceinline__ void adamw_elt(float graw, float& p, float& m, float& v, const Sc& s) {
  float g = graw * s.inv;
  g = g * s.coef;
  p = p * s.decay;
  const float d = g - m;
  m = s.small ? __builtin_fmaf(s.w1, d, m) : __builtin_fmaf(-d, s.w1c, g);
  v = v * s.b2;
  v = __builtin_fmaf(s.val2, g * g, v);
  const float den = __builtin_sqrtf(v) / s.bc2s + s.eps;
  p = __builtin_fmaf(s.nss, m / den, p);
}

// Four elements held in vector registers.
__device__ __forceinline__ void adamw4(const float (&g)[4], f4& p, f4& m, f4& v, const Sc& s) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float pk = p[k], mk = m[k], vk = v[k];
    adamw_elt(g[k], pk, mk, vk, s);
    p[k] = pk; m[k] = mk; v[k] = vk;
  }
}

template <int PD>
__device__ __forceinline__ u2 pack4(const f4& p) {
  u2 o;
  o.x = f2h<PD>(p[0]) | (f2h<PD>(p[1]) << 16);
  o.y = f2h<PD>(p[2]) | (f2h<PD>(p[3]) << 16);
  return o;
}

// ---- block reduction of a double -------------------------------------------

// One DPP lane exchange of a double (two 32-bit moves; every source lane of
// the patterns used lies in the same row, so every lane is written).
template <int kCtrl>
__device__ __forceinline__ double dpp_pair(double x) {
  const uint64_t u = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, kCtrl, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), kCtrl, 0xF, 0xF, false);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Lane i's partner i ^ 16 within each 32 lanes, through ds_swizzle (bitmask
// mode: and 0x1f, or 0, xor 0x10).
__device__ __forceinline__ double swizzle_xor16(double x) {
  constexpr int kXor16 = 0x1f | (0x10 << 10);
  const uint64_t u = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_swizzle((int)(uint32_t)u, kXor16);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_swizzle((int)(uint32_t)(u >> 32), kXor16);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Reduce over the wave with comb (commutative: comb(a, b) == comb(b, a)),
// the result in every lane. Within each row of 16 lanes through DPP:
// quad_perm for partners i ^ 1 and i ^ 2, then row_half_mirror (7 - i within
// 8) and row_mirror (15 - i within 16) in place of i ^ 4 and i ^ 8 -- by then
// every lane of a quad, then of an 8-lane half, holds the same value, so the
// mirror partner holds what the xor partner would. Across rows: ds_swizzle
// for i ^ 16, ds_bpermute for i ^ 32.
template <class Comb>
__device__ __forceinline__ double wave_reduce(double x, Comb comb) {
  x = comb(x, dpp_pair<0xb1>(x));   // quad_perm [1, 0, 3, 2]
  x = comb(x, dpp_pair<0x4e>(x));   // quad_perm [2, 3, 0, 1]
  x = comb(x, dpp_pair<0x141>(x));  // row_half_mirror
  x = comb(x, dpp_pair<0x140>(x));  // row_mirror
  x = comb(x, swizzle_xor16(x));
  x = comb(x, __shfl_xor(x, 32, 64));
  return x;
}

__device__ __forceinline__ double wave_sum(double x) {
  return wave_reduce(x, [](double a, double b) { return a + b; });
}

// Sum over the block; the result is valid in thread 0.
__device__ __forceinline__ double block_sum(double x) {
  __shared__ double lds[kWaves];
  x = wave_sum(x);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) lds[wave] = x;
  __syncthreads();
  double s = 0.0;
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s += lds[w];
  }
  return s;
}

// ---- norms other than L2 (clip_grad_norm_'s norm_type) -----------------------
// kNormSq: sum of x^2 (the L2 norm's square, as K1); kNormAbs: sum of |x|
// (p = 1); kNormMax: max |x|, NaN if any x is NaN (p = inf, as
// tensor.abs().max()); kNormPow: sum of |x|^p in fp64 (any other p > 0).
// x is the unscaled fp32 grad; every accumulation is in fp64.
enum NormKind { kNormSq = 0, kNormAbs = 1, kNormMax = 2, kNormPow = 3 };

// Commutative on what it combines (sums, or maxima of magnitudes: no -0).
template <int K>
__device__ __forceinline__ double norm_comb(double a, double b) {
  if constexpr (K == kNormMax) return (b > a || b != b) ? b : a;  // a NaN stays (b > NaN is false)
  else return a + b;
}

template <int K>
__device__ __forceinline__ double norm_acc(double acc, float x, double p) {
  if constexpr (K == kNormSq) return __builtin_fma((double)x, (double)x, acc);
  else if constexpr (K == kNormAbs) return acc + fabs((double)x);
  else if constexpr (K == kNormMax) return norm_comb<K>(acc, fabs((double)x));
  else return acc + pow(fabs((double)x), p);
}

// The elements of one 16-byte slot (8 16-bit grads or 4 fp32 grads).
template <int GD, int K>
__device__ __forceinline__ double norm_acc16(const u4& s, float inv, double p, double acc) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if constexpr (GD == DSX_F32) {
      acc = norm_acc<K>(acc, __uint_as_float(s[k]) * inv, p);
    } else {
      acc = norm_acc<K>(acc, h2f<GD>(s[k]) * inv, p);
      acc = norm_acc<K>(acc, h2f<GD>(s[k] >> 16) * inv, p);
    }
  }
  return acc;
}

// Reduce over the block with norm_comb<K>; the result is valid in thread 0.
template <int K>
__device__ __forceinline__ double block_reduce(double x) {
  __shared__ double lds[kWaves];
  x = wave_reduce(x, [](double a, double b) { return norm_comb<K>(a, b); });
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) lds[wave] = x;
  __syncthreads();
  double s = 0.0;
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s = norm_comb<K>(s, lds[w]);
  }
  return s;
}

__device__ __forceinline__ float inv_of(float scale) {
  // torch: GradScaler's inv_scale = scale.double().reciprocal().float();
  // the reference's static path multiplies by the Python double 1/loss_scale.
  return (float)(1.0 / (double)scale);
}

// ---- K1: unscale + inf/NaN + squared norm ----------------------------------
// Each element contributes (double)(f32(g) * inv)^2. The square of a finite
// fp32 value is exact in fp64 and the sum of 2^31 of them cannot overflow,
// so the sum is non-finite exactly when some unscaled grad is inf or NaN.
//
// fold != NULL (the same state) starts a two-launch step whose finalize runs
// inside K2 (k2_adamw_fold): block 0 records the entry scale and t with the
// one-shot clip flag, which it consumes, in step_scale / step_t2. The K2
// blocks read those two fields, which nothing else writes during the step,
// while one of them writes the state's updated fields.

template <int GD, int U, bool NT>
__global__ __launch_bounds__(kBlock) void k1_unscale_norm(const void* __restrict__ gv, int64_t n,
                                                          const DsxState* state, double* __restrict__ partials,
                                                          DsxState* fold) {
  using G = Grad<GD>;
  const float inv = inv_of(state->scale);
  if (fold != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
    const int32_t armed = fold->clip_once != 0 ? 1 : 0;
    fold->step_scale = fold->scale;
    fold->step_t2 = 2 * fold->t + armed;
    fold->clip_once = 0;
  }
  const u4* g16 = static_cast<const u4*>(gv);
  const typename G::elem* g = static_cast<const typename G::elem*>(gv);
  const int64_t nvec = n / G::per16;
  const int64_t stride = (int64_t)gridDim.x * kBlock * U;
  double acc = 0.0;
  for (int64_t i0 = (int64_t)blockIdx.x * kBlock * U + threadIdx.x; i0 < nvec; i0 += stride) {
    u4 S[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + (int64_t)u * kBlock;
      S[u] = (i < nvec) ? ld<NT>(g16 + i) : u4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc = G::sumsq16(S[u], inv, acc);
  }
  const int64_t tail0 = nvec * G::per16;
  const int64_t gt = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (gt < n - tail0) {
    const float a = G::one(g[tail0 + gt]) * inv;
    acc = __builtin_fma((double)a, (double)a, acc);
  }
  const double s = block_sum(acc);
  if (threadIdx.x == 0) partials[blockIdx.x] = s;
}

// ---- K1 for clip_grad_norm_'s norm types -----------------------------------
// The same pass as K1 with the per-element term and the block combine of
// NormKind K: per-block partials of sum |x|^p (or max |x|), x = f32(g) * inv.

template <int GD, int K>
__global__ __launch_bounds__(kBlock) void k1_norm(const void* __restrict__ gv, int64_t n,
                                                  const DsxState* __restrict__ state, double p,
                                                  double* __restrict__ partials) {
  using G = Grad<GD>;
  constexpr int U = 4;
  const float inv = inv_of(state->scale);
  const u4* g16 = static_cast<const u4*>(gv);
  const typename G::elem* g = static_cast<const typename G::elem*>(gv);
  const int64_t nvec = n / G::per16;
  const int64_t stride = (int64_t)gridDim.x * kBlock * U;
  double acc = 0.0;
  for (int64_t i0 = (int64_t)blockIdx.x * kBlock * U + threadIdx.x; i0 < nvec; i0 += stride) {
    u4 S[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + (int64_t)u * kBlock;
      S[u] = (i < nvec) ? ld<true>(g16 + i) : u4{0u, 0u, 0u, 0u};  // zeros add nothing to any kind
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc = norm_acc16<GD, K>(S[u], inv, p, acc);
  }
  const int64_t tail0 = nvec * G::per16;
  const int64_t gt = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (gt < n - tail0) acc = norm_acc<K>(acc, G::one(g[tail0 + gt]) * inv, p);
  const double s = block_reduce<K>(acc);
  if (threadIdx.x == 0) partials[blockIdx.x] = s;
}

template <int GD, int K>
__global__ __launch_bounds__(kBlock) void k1_norm_multi(const DsxTensorRef* __restrict__ tensors,
                                                        const DsxChunk* __restrict__ chunks, int64_t nchunks,
                                                        const DsxState* __restrict__ state, double p,
                                                        double* __restrict__ partials) {
  using G = Grad<GD>;
  constexpr int U = 4;
  const float inv = inv_of(state->scale);
  double acc = 0.0;
  for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const DsxChunk ch = chunks[c];
    const typename G::elem* g = static_cast<const typename G::elem*>(tensors[ch.tensor].grad) + ch.start;
    const int64_t len = ch.len;
    int64_t done = 0;
    if (aligned16(g)) {
      const u4* g16 = reinterpret_cast<const u4*>(g);
      const int64_t nvec = len / G::per16;
      for (int64_t i0 = threadIdx.x; i0 < nvec; i0 += kBlock * U) {
        u4 S[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t i = i0 + (int64_t)u * kBlock;
          S[u] = (i < nvec) ? ld<true>(g16 + i) : u4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc = norm_acc16<GD, K>(S[u], inv, p, acc);
      }
      done = nvec * G::per16;
    }
    for (int64_t e = done + threadIdx.x; e < len; e += kBlock) acc = norm_acc<K>(acc, G::one(g[e]) * inv, p);
  }
  const double s = block_reduce<K>(acc);
  if (threadIdx.x == 0) partials[blockIdx.x] = s;
}

// clip_grad_norm_'s decision, one block: the partials of NormKind K -> the
// norm (sqrt for p = 2, total^(1/p) for other finite p, the total itself for
// p = 1 and p = inf) into *norm_out, and the coefficient the next K0 applies
// instead of the configured clip: max_norm / (norm + clip_eps) in double,
// rounded to fp32, iff norm > max_norm (Src/zero/utils.py:209-214), else 1.
template <int K>
__global__ __launch_bounds__(kBlock) void k_clip_prepare(const double* __restrict__ partials, int32_t nparts,
                                                         double p, double max_norm, double clip_eps,
                                                         DsxState* __restrict__ state, double* __restrict__ norm_out) {
  double x = 0.0;
  for (int i = threadIdx.x; i < nparts; i += kBlock) x = norm_comb<K>(x, partials[i]);
  const double total = block_reduce<K>(x);
  if (threadIdx.x != 0) return;
  double norm = total;
  if constexpr (K == kNormSq) norm = sqrt(total);
  else if constexpr (K == kNormPow) norm = pow(total, 1.0 / p);
  float coef = 1.0f;
  if (norm > max_norm) coef = (float)(max_norm / (norm + clip_eps));
  *norm_out = norm;
  state->clip_once_coef = coef;
  state->clip_once = 1;
}

// ---- K1 folded into a grad copy ---------------------------------------------------
// The flat form's post-accumulate hook copies the grad autograd produced into
// the flat buffer. This kernel makes that copy and does K1's work for the
// copied elements on the way: one fp64 partial of (f32(g) * inv)^2 per block,
// exactly as k1_unscale_norm sums them. k_reduce_segments then turns each
// parameter's block partials into one partial, in a fixed order, so that K0
// can finalize from one partial per parameter instead of a K1 pass over the
// whole buffer.

template <int GD, int U>
__global__ __launch_bounds__(kBlock) void k1_copy_unscale_norm(const void* __restrict__ src, void* __restrict__ dst,
                                                               int64_t n, const DsxState* __restrict__ state,
                                                               double* __restrict__ partials) {
  using G = Grad<GD>;
  using E = typename G::elem;
  const float inv = inv_of(state->scale);
  const u4* s16 = static_cast<const u4*>(src);
  u4* d16 = static_cast<u4*>(dst);
  const E* se = static_cast<const E*>(src);
  E* de = static_cast<E*>(dst);
  const int64_t nvec = n / G::per16;
  const int64_t stride = (int64_t)gridDim.x * kBlock * U;
  double acc = 0.0;
  for (int64_t i0 = (int64_t)blockIdx.x * kBlock * U + threadIdx.x; i0 < nvec; i0 += stride) {
    u4 S[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + (int64_t)u * kBlock;
      S[u] = (i < nvec) ? ld<true>(s16 + i) : u4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + (int64_t)u * kBlock;
      if (i < nvec) st<true>(d16 + i, S[u]);
      acc = G::sumsq16(S[u], inv, acc);
    }
  }
  const int64_t tail0 = nvec * G::per16;
  const int64_t gt = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (gt < n - tail0) {
    const E e = se[tail0 + gt];
    de[tail0 + gt] = e;
    const float a = G::one(e) * inv;
    acc = __builtin_fma((double)a, (double)a, acc);
  }
  const double s = block_sum(acc);
  if (threadIdx.x == 0) partials[blockIdx.x] = s;
}

// out[b] = sum of partials[offsets[b] .. offsets[b + 1]), by block b, each
// thread over a fixed stride and the block reduce in a fixed tree: the same
// bits for the same partials.
__global__ __launch_bounds__(kBlock) void k_reduce_segments(const double* __restrict__ partials,
                                                            const int64_t* __restrict__ offsets,
                                                            double* __restrict__ out) {
  const int64_t lo = offsets[blockIdx.x], hi = offsets[blockIdx.x + 1];
  double acc = 0.0;
  for (int64_t i = lo + threadIdx.x; i < hi; i += kBlock) acc += partials[i];
  const double s = block_sum(acc);
  if (threadIdx.x == 0) out[blockIdx.x] = s;
}

// ---- K0: finalize ------------------------------------------------------------

// Hyper-parameters a device-resident group block may hold: the admissible
// ranges of torch.optim.Adam's constructor, checked again on the device for
// the graph path (where the host cannot see the values at launch).
__device__ __forceinline__ bool hyper_ok(const DsxAdamwHyper& h) {
  return h.lr >= 0.0 && h.eps >= 0.0 && h.beta1 >= 0.0 && h.beta1 < 1.0 && h.beta2 >= 0.0 && h.beta2 < 1.0 &&
         h.weight_decay >= 0.0 && h.clip_eps >= 0.0 && h.max_grad_norm == h.max_grad_norm;
}

// The step's decision from the squared norm and the state as the step began
// (scale, t, clip_once, clip_once_coef): norm, skip, clip coefficient, t.
// Error bits found on the way are set in s.error.
struct Decision {
  double norm;
  float inv, coef;
  int32_t t;  // t of a step that is not skipped
  int ng;     // live groups (0 when the group inputs are bad)
  bool found_inf, skip;
};

__device__ Decision decide(double sumsq, DsxState& s, const DsxGroupsDev& grp, bool groups_bad) {
  Decision d;
  d.norm = sqrt(sumsq);
  d.inv = inv_of(s.scale);
  d.found_inf = !__builtin_isfinite(sumsq);
  d.t = s.t + 1;
  d.skip = d.found_inf || groups_bad;
  if (groups_bad) s.error |= DSX_STATE_ERR_GROUPS;
  d.ng = groups_bad ? 0 : grp.ngroups;
  if (!d.skip) {
    for (int k = 0; k < d.ng; ++k) {
      const int32_t tk = d.t - grp.t_offset[k];
      if (tk < 1 || tk > grp.bc_len) {
        d.skip = true;
        s.error |= DSX_STATE_ERR_BC_TABLE;
      }
    }
  }
  // A coefficient armed by clip_grad_norm_ (dsx_clip_prepare) replaces the
  // configured clip for this one step, applied or skipped, and is consumed.
  d.coef = 1.0f;
  if (d.ng > 0 && !d.skip) {
    const DsxAdamwHyper& h0 = grp.hyper[0];
    if (s.clip_once)
      d.coef = s.clip_once_coef;
    else if (h0.max_grad_norm > 0.0 && d.norm > h0.max_grad_norm)
      d.coef = (float)(h0.max_grad_norm / (d.norm + h0.clip_eps));
  }
  return d;
}

// Group k's fp32 step scalars. Slots at or past the live groups get skip = 1,
// so a K2 launched for them leaves its group unchanged rather than reusing an
// older step's scalars.
__device__ __forceinline__ DsxStepScalars record_bc(const Decision& d, const DsxState& s, const DsxGroupsDev& grp,
                                                    int k, double sumsq, double bc1, double bc2s) {
  const bool live = k < d.ng;
  DsxStepScalars o = {};
  o.sumsq = sumsq;
  o.norm = d.norm;
  o.inv_scale = d.inv;
  o.clip_coef = d.coef;
  o.decay = 1.0f;
  o.skip = (d.skip || !live) ? 1 : 0;
  o.t = (d.skip ? s.t : d.t) - (live ? grp.t_offset[k] : 0);
  if (!d.skip && live) {
    const DsxAdamwHyper& hp = grp.hyper[k];
    if (hp.weight_decay != 0.0) o.decay = (float)(1.0 - hp.lr * hp.weight_decay);
    o.w1 = (float)(1.0 - hp.beta1);
    o.w1c = 1.0f - o.w1;
    o.b2 = (float)hp.beta2;
    o.val2 = (float)(1.0 - hp.beta2);
    o.eps = (float)hp.eps;
    o.bc2s = (float)bc2s;
    o.nss = (float)(-(hp.lr / bc1));
  }
  return o;
}

// Group k's bias corrections for step t (1-based), or (1, 1) when t is out
// of the table's range (decide() then skips the step). The table is read
// through the constant address space, i.e. with scalar loads (t and k are
// uniform; no kernel writes a bias-correction table).
typedef const double __attribute__((address_space(4)))* ConstDoubles;

__device__ __forceinline__ void bc_of(const DsxGroupsDev& grp, int k, int32_t t, double& bc1, double& bc2s) {
  const int32_t tk = t - grp.t_offset[k];
  bc1 = 1.0;
  bc2s = 1.0;
  if (tk >= 1 && tk <= grp.bc_len) {
    const ConstDoubles row = (ConstDoubles)(uintptr_t)(grp.bc_table[k] + 2 * (int64_t)(tk - 1));
    bc1 = row[0];
    bc2s = row[1];
  }
}

__device__ DsxStepScalars record(const Decision& d, const DsxState& s, const DsxGroupsDev& grp, int k,
                                 double sumsq) {
  double bc1 = 1.0, bc2s = 1.0;
  if (!d.skip && k < d.ng) bc_of(grp, k, d.t, bc1, bc2s);
  return record_bc(d, s, grp, k, sumsq, bc1, bc2s);
}

// The state after the step: counters, t, the loss scaler, the step's record
// fields, and the entry values step_scale / step_t2.
__device__ void advance(const Decision& d, DsxState& s, const DsxScalerConfig& scfg) {
  const bool dynamic = scfg.mode == DSX_SCALE_DYNAMIC;
  s.step_scale = s.scale;
  s.step_t2 = 2 * s.t + (s.clip_once != 0 ? 1 : 0);
  s.clip_once = 0;
  if (d.found_inf) {
    s.overflow_count += 1;
    if (dynamic) {
      if (scfg.hysteresis <= 1 || s.hyst_left <= 1) {
        const float next = s.scale * scfg.backoff_factor;
        s.scale = next > scfg.min_scale ? next : scfg.min_scale;
      } else {
        s.hyst_left -= 1;
      }
      s.good_steps = 0;
    }
  } else if (!d.skip) {
    s.t = d.t;
    if (dynamic) {
      s.good_steps += 1;
      if (s.good_steps >= scfg.window) {
        const float next = s.scale * scfg.growth_factor;
        if (__builtin_isfinite(next)) s.scale = next;
        s.good_steps = 0;
        s.hyst_left = scfg.hysteresis;
      }
    }
  }
  s.iter += 1;
  s.last_skip = d.skip ? 1 : 0;
  s.last_norm = d.norm;
}

// A group block read from device memory fails these checks when its group
// count is out of range or a group's inputs are (the host cannot check it at
// launch in the graph form).
__device__ __forceinline__ bool groups_bad_dev(const DsxGroupsDev& grp, int32_t max_groups) {
  bool bad = grp.ngroups < 1 || grp.ngroups > max_groups || grp.ngroups > DSX_MAX_GROUPS || grp.bc_len < 0;
  for (int k = 0; !bad && k < grp.ngroups; ++k)
    bad = !hyper_ok(grp.hyper[k]) || grp.t_offset[k] < 0 || (grp.bc_len > 0 && grp.bc_table[k] == nullptr);
  return bad;
}

// Thread 0 only. Global part of a step (norm, skip, clip, t, scaler) once;
// per-group fp32 scalars into out[0..nout).
__device__ void finalize_body(double sumsq, DsxState* __restrict__ state, const DsxScalerConfig& scfg,
                              const DsxGroupsDev& grp, bool groups_bad, int nout,
                              DsxStepScalars* __restrict__ out) {
  DsxState s = *state;
  const Decision d = decide(sumsq, s, grp, groups_bad);
  for (int k = 0; k < nout; ++k) out[k] = record(d, s, grp, k, sumsq);
  advance(d, s, scfg);
  *state = s;
}

__device__ __forceinline__ double reduce_partials(const double* __restrict__ partials, int32_t nparts) {
  double x = 0.0;
  for (int i = threadIdx.x; i < nparts; i += kBlock) x += partials[i];
  return block_sum(x);
}

// Group inputs as a kernel argument (validated on the host).
__global__ __launch_bounds__(kBlock) void k0_finalize(const double* __restrict__ partials, int32_t nparts,
                                                      DsxState* __restrict__ state, DsxScalerConfig scfg,
                                                      DsxGroupsDev grp, DsxStepScalars* __restrict__ out) {
  const double sumsq = reduce_partials(partials, nparts);
  if (threadIdx.x == 0) finalize_body(sumsq, state, scfg, grp, false, grp.ngroups, out);
}

// Group inputs from device memory (the graph path); validated here.
__global__ __launch_bounds__(kBlock) void k0_finalize_dev(const double* __restrict__ partials, int32_t nparts,
                                                          DsxState* __restrict__ state, DsxScalerConfig scfg,
                                                          const DsxGroupsDev* __restrict__ gp, int32_t max_groups,
                                                          DsxStepScalars* __restrict__ out) {
  const double sumsq = reduce_partials(partials, nparts);
  if (threadIdx.x != 0) return;
  // read in place: a copy of the 1112-byte block would live in scratch memory
  const DsxGroupsDev& grp = *gp;
  finalize_body(sumsq, state, scfg, grp, groups_bad_dev(grp, max_groups), max_groups, out);
}

// Writes a group block passed by value (through the kernel-argument
// segment, so no DMA copy and no host staging buffer) to device memory,
// 8 bytes per lane.
__global__ __launch_bounds__(64) void k_store_groups(DsxGroupsDev g, DsxGroupsDev* __restrict__ dst) {
  static_assert(sizeof(DsxGroupsDev) % 8 == 0, "DsxGroupsDev is stored in 8-byte words");
  const uint64_t* src = reinterpret_cast<const uint64_t*>(&g);
  uint64_t* out = reinterpret_cast<uint64_t*>(dst);
  for (int i = threadIdx.x; i < (int)(sizeof(DsxGroupsDev) / 8); i += 64) out[i] = src[i];
}

__global__ void k_state_init(DsxState* state, float scale, int32_t hysteresis) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    DsxState s = {};
    s.scale = scale;
    s.hyst_left = hysteresis;
    *state = s;
  }
}

// ---- K2: AdamW + cast over a flat partition ----------------------------------

// The slot loop of K2. MATH = false is the traffic probe: the same loads,
// stores, cast and launch shape with the AdamW math left out, so that K2 can
// be timed against its own access pattern (the values written back are the
// ones read, and p16 gets the cast of the unchanged master).
template <int GD, int PD, int U, bool NT, bool DRAIN, bool MATH>
__device__ __forceinline__ void k2_flat_body(float* __restrict__ p, float* __restrict__ m, float* __restrict__ v,
                                             uint16_t* __restrict__ p16, const void* __restrict__ gv, int64_t n,
                                             const DsxStepScalars* __restrict__ scp) {
  using G = Grad<GD>;
  using GS = typename G::slot4;
  Sc s = {};
  if constexpr (MATH) {
    if (scp->skip) return;
    s = load_sc(*scp);
  }
  f4* p4 = reinterpret_cast<f4*>(p);
  f4* m4 = reinterpret_cast<f4*>(m);
  f4* v4 = reinterpret_cast<f4*>(v);
  u2* o2 = reinterpret_cast<u2*>(p16);
  const GS* g4 = static_cast<const GS*>(gv);
  const typename G::elem* g = static_cast<const typename G::elem*>(gv);
  const bool cast = p16 != nullptr;
  const int64_t nvec = n >> 2;  // 4 elements per slot
  const int64_t stride = (int64_t)gridDim.x * kBlock * U;
  for (int64_t i0 = (int64_t)blockIdx.x * kBlock * U + threadIdx.x; i0 < nvec; i0 += stride) {
    GS Gs[U];
    f4 P[U], M[U], V[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + (int64_t)u * kBlock;
      if (i < nvec) {
        // exp_avg_sq, exp_avg, master, grad: this order, and the stores in
        // the reverse of theirs below, measured 0.5% faster on the headline
        // shard than grad-first loads and master-first stores
        V[u] = ld<NT>(v4 + i);
        M[u] = ld<NT>(m4 + i);
        P[u] = ld<NT>(p4 + i);
        Gs[u] = ld<NT>(g4 + i);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + (int64_t)u * kBlock;
      if (i < nvec) {
        f4 pp = P[u], mm = M[u], vv = V[u];
        if constexpr (MATH) {
          float gf[4];
          G::four(Gs[u], gf);
          adamw4(gf, pp, mm, vv, s);
        } else {
          // opaque to the compiler: every load and store stays, as in K2
          asm volatile("" : "+v"(pp), "+v"(mm), "+v"(vv) : "v"(Gs[u]));
        }
        if (cast) st<NT>(o2 + i, pack4<PD>(pp));
        st<NT>(v4 + i, vv);
        st<NT>(m4 + i, mm);
        st<NT>(p4 + i, pp);
      }
    }
    // Drain: this wave's stores complete before its next loads issue. Fewer
    // requests in flight chip-wide keep DRAM's read/write mix efficient.
    if constexpr (DRAIN) __builtin_amdgcn_s_waitcnt(0);
  }
  const int64_t tail0 = nvec << 2;
  const int64_t gt = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (gt < n - tail0) {
    const int64_t e = tail0 + gt;
    float pe = p[e], me = m[e], ve = v[e];
    if constexpr (MATH) {
      adamw_elt(G::one(g[e]), pe, me, ve, s);
    } else {
      asm volatile("" : "+v"(pe), "+v"(me), "+v"(ve) : "v"(G::one(g[e])));
    }
    p[e] = pe; m[e] = me; v[e] = ve;
    if (cast) p16[e] = (uint16_t)f2h<PD>(pe);
  }
}

template <int GD, int PD, int U, bool NT, bool DRAIN>
__global__ __launch_bounds__(kBlock) void k2_adamw_flat(float* __restrict__ p, float* __restrict__ m,
                                                        float* __restrict__ v, uint16_t* __restrict__ p16,
                                                        const void* __restrict__ gv, int64_t n,
                                                        const DsxStepScalars* __restrict__ scp) {
  k2_flat_body<GD, PD, U, NT, DRAIN, true>(p, m, v, p16, gv, n, scp);
}

template <int GD, int PD, int U, bool NT, bool DRAIN>
__global__ __launch_bounds__(kBlock) void k2_traffic_probe(float* __restrict__ p, float* __restrict__ m,
                                                           float* __restrict__ v, uint16_t* __restrict__ p16,
                                                           const void* __restrict__ gv, int64_t n,
                                                           const DsxStepScalars* __restrict__ scp) {
  k2_flat_body<GD, PD, U, NT, DRAIN, false>(p, m, v, p16, gv, n, scp);
}

// ---- K2 with the finalize folded in (two-launch step) ---------------------------
// After a K1 launched with fold (block 0 recorded the entry scale, t and the
// one-shot clip flag in step_scale / step_t2), every thread of this kernel
// runs K0's decision itself: the same reduction of K1's partials
// (reduce_partials' per-thread order and block_sum's tree, so the same bits)
// and the same decide / record code on the entry values, giving the scalars
// K0 would give. The launch with `writer` set (the step's first K2 launch)
// has one more block, its last, which does no slot work: it reduces the
// partials and decides the same way, then writes every group's record to
// out[] and the state's updated fields, leaving step_scale / step_t2 and
// clip_once_coef, the fields the other blocks read, untouched. (A block of
// its own keeps that code's registers out of the slot blocks' path.) No block waits for another and nothing is counted
// across blocks. Each thread issues its partials' loads first and its first
// trip's slot loads next, so that waiting for the partials does not wait for
// the slot loads, which stay in flight while the block reduces and decides;
// the entry values and the bias corrections come through scalar loads, which
// wait on neither. 1 <= nparts <= kFoldMaxParts (two partials per thread),
// n >= 4.
constexpr int kFoldParts = 2;
constexpr int kFoldMaxParts = kFoldParts * kBlock;

// block_sum's tree with its result in every thread (each adds the wave sums
// in the order thread 0 does).
__device__ __forceinline__ double block_sum_all(double x) {
  __shared__ double lds[kWaves];
  x = wave_sum(x);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) lds[wave] = x;
  __syncthreads();
  double s = 0.0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) s += lds[w];
  return s;
}

// The step scalars, equal in every lane, moved to scalar registers (so that
// the slot loop holds them as K2 does, where they come from scalar loads).
__device__ __forceinline__ float sgpr(float x) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}

__device__ __forceinline__ Sc uniform_sc(const Sc& a) {
  Sc r;
  r.inv = sgpr(a.inv); r.coef = sgpr(a.coef); r.decay = sgpr(a.decay);
  r.w1 = sgpr(a.w1); r.w1c = sgpr(a.w1c); r.b2 = sgpr(a.b2); r.val2 = sgpr(a.val2);
  r.eps = sgpr(a.eps); r.bc2s = sgpr(a.bc2s); r.nss = sgpr(a.nss);
  r.small = __builtin_amdgcn_readfirstlane(a.small ? 1 : 0) != 0;
  return r;
}

// The group block gb: a DsxGroupsDev kernel argument checked on the host
// (the eager form; the writer writes its ngroups records), or a pointer to
// the block in device memory (the graph form), checked here as
// k0_finalize_dev checks it -- a bad block skips the step with
// DSX_STATE_ERR_GROUPS set -- with records for max_groups slots. (One kernel
// template for both, with the body inline: as a shared function the compiler
// gave it more registers than K2's occupancy allows.)
__device__ __forceinline__ const DsxGroupsDev& group_block(const DsxGroupsDev& g) { return g; }
__device__ __forceinline__ const DsxGroupsDev& group_block(const DsxGroupsDev* g) { return *g; }

template <int GD, int PD, int U, bool NT, typename GB>
__global__ __launch_bounds__(kBlock) void k2_adamw_fold(float* __restrict__ p, float* __restrict__ m,
                                                        float* __restrict__ v, uint16_t* __restrict__ p16,
                                                        const void* __restrict__ gv, int64_t n,
                                                        const double* __restrict__ partials, int32_t nparts,
                                                        DsxState* state, DsxScalerConfig scfg, GB gb,
                                                        int32_t max_groups, int32_t group, int32_t writer,
                                                        DsxStepScalars* __restrict__ out) {
  constexpr bool DEV = std::is_pointer<GB>::value;
  const DsxGroupsDev& grp = group_block(gb);
  const bool groups_bad = DEV ? groups_bad_dev(grp, max_groups) : false;
  const int nout = DEV ? max_groups : grp.ngroups;
  using G = Grad<GD>;
  using GS = typename G::slot4;
  if (writer && blockIdx.x == gridDim.x - 1) {
    // The extra block of the writing launch: the step's records and state.
    double x = 0.0;
    for (int i = threadIdx.x; i < nparts; i += kBlock) x += partials[i];
    const double sumsq = block_sum_all(x);
    if (threadIdx.x == 0) {
      DsxState f = *state;
      const int32_t t2 = f.step_t2;
      f.clip_once = t2 & 1;  // K1 consumed the live flag into step_t2
      const Decision d = decide(sumsq, f, grp, groups_bad);
      for (int k = 0; k < nout; ++k) out[k] = record(d, f, grp, k, sumsq);
      advance(d, f, scfg);
      state->scale = f.scale;
      state->good_steps = f.good_steps;
      state->hyst_left = f.hyst_left;
      state->t = f.t;
      state->iter = f.iter;
      state->overflow_count = f.overflow_count;
      state->error = f.error;
      state->last_skip = f.last_skip;
      state->last_norm = f.last_norm;
      state->clip_once = 0;
    }
    return;
  }
  // The entry values, read first (vector loads: `state` is written below).
  int32_t t2 = state->step_t2;
  float scale0 = state->step_scale, coef1 = state->clip_once_coef;
  // Every vector load below is issued unconditionally (an index past the end
  // reads the last element again, and the value is not used), so the number
  // of loads in flight is the same on every path and waiting for the
  // partials waits for them alone.
  double pv[kFoldParts];
#pragma unroll
  for (int j = 0; j < kFoldParts; ++j) {
    const int i = threadIdx.x + j * kBlock;
    const double x = partials[i < nparts ? i : nparts - 1];
    pv[j] = i < nparts ? x : 0.0;
  }
  f4* p4 = reinterpret_cast<f4*>(p);
  f4* m4 = reinterpret_cast<f4*>(m);
  f4* v4 = reinterpret_cast<f4*>(v);
  u2* o2 = reinterpret_cast<u2*>(p16);
  const GS* g4 = static_cast<const GS*>(gv);
  const typename G::elem* g = static_cast<const typename G::elem*>(gv);
  const bool cast = p16 != nullptr;
  const int64_t nvec = n >> 2;
  const int64_t stride = (int64_t)(gridDim.x - (writer ? 1 : 0)) * kBlock * U;  // the slot blocks
  int64_t i0 = (int64_t)blockIdx.x * kBlock * U + threadIdx.x;
  GS Gs[U];
  f4 P[U], M[U], V[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    int64_t i = i0 + (int64_t)u * kBlock;
    i = i < nvec ? i : nvec - 1;  // nvec >= 1 (n >= 4 on this path)
    Gs[u] = ld<NT>(g4 + i);
    P[u] = ld<NT>(p4 + i);
    M[u] = ld<NT>(m4 + i);
    V[u] = ld<NT>(v4 + i);
  }
  // After the slot loads are issued: the entry values (the oldest loads, so
  // waiting for them waits for nothing else), then this group's bias
  // corrections for t + 1 through scalar loads.
  asm volatile("" : "+v"(t2), "+v"(scale0), "+v"(coef1));
  DsxState s = {};
  s.scale = scale0;
  t2 = __builtin_amdgcn_readfirstlane(t2);
  s.t = t2 >> 1;
  s.clip_once = t2 & 1;
  s.clip_once_coef = coef1;
  double bc1 = 1.0, bc2s = 1.0;
  if (!groups_bad && group < grp.ngroups) bc_of(grp, group, s.t + 1, bc1, bc2s);
  // The slot loads issue before the first use of a partial.
  asm volatile("" : "+v"(pv[0]), "+v"(pv[1]));
  // reduce_partials' order: each thread adds its partials in index order
  // (the zeros past nparts add nothing to a sum of squares), then the tree.
  double x = 0.0;
#pragma unroll
  for (int j = 0; j < kFoldParts; ++j) x += pv[j];
  const double sumsq = block_sum_all(x);
  const Decision d = decide(sumsq, s, grp, groups_bad);
  // This group is skipped with the step, or when it is past the block's live
  // groups (a device block may hold fewer than the plan): record()'s skip.
  if (!d.skip && group < d.ng) {
    const Sc sc = uniform_sc(load_sc(record_bc(d, s, grp, group, sumsq, bc1, bc2s)));
    for (;;) {
      // Every slot's loads are taken in here, on every path, as in K3's
      // chunk loop: a slot past the end would otherwise leave its loads
      // pending into the next trip, whose register writes would then wait for
      // this trip's stores too.
#pragma unroll
      for (int u = 0; u < U; ++u) asm volatile("" : "+v"(Gs[u]), "+v"(P[u]), "+v"(M[u]), "+v"(V[u]));
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = i0 + (int64_t)u * kBlock;
        if (i < nvec) {
          float gf[4];
          G::four(Gs[u], gf);
          f4 pp = P[u], mm = M[u], vv = V[u];
          adamw4(gf, pp, mm, vv, sc);
          st<NT>(p4 + i, pp);
          st<NT>(m4 + i, mm);
          st<NT>(v4 + i, vv);
          if (cast) st<NT>(o2 + i, pack4<PD>(pp));
        }
      }
      i0 += stride;
      if (i0 >= nvec) break;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int64_t i = i0 + (int64_t)u * kBlock;
        i = i < nvec ? i : nvec - 1;
        Gs[u] = ld<NT>(g4 + i);
        P[u] = ld<NT>(p4 + i);
        M[u] = ld<NT>(m4 + i);
        V[u] = ld<NT>(v4 + i);
      }
    }
    const int64_t tail0 = nvec << 2;
    const int64_t gt = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (gt < n - tail0) {
      const int64_t e = tail0 + gt;
      float pe = p[e], me = m[e], ve = v[e];
      adamw_elt(G::one(g[e]), pe, me, ve, sc);
      p[e] = pe; m[e] = me; v[e] = ve;
      if (cast) p16[e] = (uint16_t)f2h<PD>(pe);
    }
  }
}

// ---- K3: ragged lists ----------------------------------------------------------

// Chunk and tensor records (kernel-invariant: the host or an earlier launch
// wrote them), read through the constant address space: scalar loads, and
// the pointers a tensor record holds are then known to address global
// memory, so a chunk's slot accesses compile to global loads and stores,
// counted by vmcnt alone (flat ones also count on lgkmcnt, which ties every
// wait for a scalar record to the stores still in flight).
typedef const DsxChunk __attribute__((address_space(4)))* ConstChunk;
typedef const DsxTensorRef __attribute__((address_space(4)))* ConstTensorRef;
typedef const DsxStepScalars __attribute__((address_space(4)))* ConstScalars;

__device__ __forceinline__ DsxChunk chunk_rec(const DsxChunk* chunks, int64_t c) {
  const ConstChunk cc = (ConstChunk)(uintptr_t)(chunks + c);
  DsxChunk ch;
  ch.tensor = cc->tensor;
  ch.reserved = 0;
  ch.start = cc->start;
  ch.len = cc->len;
  return ch;
}

__device__ __forceinline__ DsxTensorRef tensor_rec(const DsxTensorRef* tensors, int32_t t) {
  const ConstTensorRef ct = (ConstTensorRef)(uintptr_t)(tensors + t);
  DsxTensorRef tr;
  tr.master = ct->master;
  tr.exp_avg = ct->exp_avg;
  tr.exp_avg_sq = ct->exp_avg_sq;
  tr.param16 = ct->param16;
  tr.grad = ct->grad;
  tr.numel = ct->numel;
  tr.group = ct->group;
  tr.reserved = 0;
  return tr;
}

__device__ __forceinline__ Sc scalars_rec(const DsxStepScalars* scalars, int32_t group) {
  const ConstScalars cs = (ConstScalars)(uintptr_t)(scalars + group);
  Sc r;
  r.inv = cs->inv_scale; r.coef = cs->clip_coef; r.decay = cs->decay;
  r.w1 = cs->w1; r.w1c = cs->w1c; r.b2 = cs->b2; r.val2 = cs->val2;
  r.eps = cs->eps; r.bc2s = cs->bc2s; r.nss = cs->nss;
  r.small = fabsf(r.w1) < 0.5f;
  return r;
}

// K1 over a chunk table. Block b reduces chunks b, b + grid, ... in order,
// each as K1's slot loop (four 16-byte loads per thread in flight before any
// use) when its grad is 16-byte aligned, element by element otherwise. With
// WAVE, each wave takes its own chunks (wave w of block b: chunks 4b + w,
// 4b + w + 4 grid, ...): for tables of small chunks, where a block's 256
// threads would leave most of a trip empty (a 2048-element 16-bit chunk is
// one trip of one wave). The next chunk's record is requested with the
// current chunk's tensor record, so that it is in by the time the current
// chunk is done.
template <int GD, bool WAVE>
__global__ __launch_bounds__(kBlock) void k1_unscale_norm_multi(const DsxTensorRef* __restrict__ tensors,
                                                                const DsxChunk* __restrict__ chunks,
                                                                int64_t nchunks, const DsxState* state,
                                                                double* __restrict__ partials, DsxState* fold) {
  using G = Grad<GD>;
  constexpr int U = 4;
  constexpr int kWaves = kBlock / 64;
  constexpr int kLanes = WAVE ? 64 : kBlock;
  const float inv = inv_of(state->scale);
  if (fold != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {  // as k1_unscale_norm
    const int32_t armed = fold->clip_once != 0 ? 1 : 0;
    fold->step_scale = fold->scale;
    fold->step_t2 = 2 * fold->t + armed;
    fold->clip_once = 0;
  }
  double acc = 0.0;
  const int lane = WAVE ? (int)(threadIdx.x & 63) : (int)threadIdx.x;
  const int64_t stride = WAVE ? (int64_t)gridDim.x * kWaves : (int64_t)gridDim.x;
  int64_t c = WAVE ? (int64_t)blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)
                   : (int64_t)blockIdx.x;
  if (c < nchunks) {  // the grid is the partial count, which may exceed the chunk count
    DsxChunk ch = chunk_rec(chunks, c);
    for (;;) {
      const typename G::elem* g = static_cast<const typename G::elem*>(tensor_rec(tensors, ch.tensor).grad) + ch.start;
      const int64_t cn = c + stride;
      const DsxChunk chn = chunk_rec(chunks, cn < nchunks ? cn : c);
      int64_t done = 0;
      if (aligned16(g)) {
        const u4* g16 = reinterpret_cast<const u4*>(g);
        const int64_t nvec = ch.len / G::per16;
        for (int64_t i0 = lane; i0 < nvec; i0 += kLanes * U) {
          u4 S[U];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + (int64_t)u * kLanes;
            S[u] = (i < nvec) ? ld<true>(g16 + i) : u4{0u, 0u, 0u, 0u};
          }
#pragma unroll
          for (int u = 0; u < U; ++u) acc = G::sumsq16(S[u], inv, acc);
        }
        done = nvec * G::per16;
      }
      for (int64_t e = done + lane; e < ch.len; e += kLanes) {
        const float a = G::one(g[e]) * inv;
        acc = __builtin_fma((double)a, (double)a, acc);
      }
      if (cn >= nchunks) break;
      c = cn;
      ch = chn;
    }
  }
  const double s = block_sum(acc);
  if (threadIdx.x == 0) partials[blockIdx.x] = s;
}

// One chunk's arrays, and whether every one is aligned for its 4-element slot
// (vec: the K2 slot loop; otherwise element by element).
template <int GD>
struct ChunkView {
  float* p;
  float* m;
  float* v;
  uint16_t* p16;
  const typename Grad<GD>::elem* g;
  int64_t len, nvec;
  bool vec;
};

template <int GD>
__device__ __forceinline__ ChunkView<GD> chunk_view(const DsxTensorRef& tr, const DsxChunk& ch) {
  using G = Grad<GD>;
  ChunkView<GD> c;
  c.p = tr.master + ch.start;
  c.m = tr.exp_avg + ch.start;
  c.v = tr.exp_avg_sq + ch.start;
  c.p16 = tr.param16 ? static_cast<uint16_t*>(tr.param16) + ch.start : nullptr;
  c.g = static_cast<const typename G::elem*>(tr.grad) + ch.start;
  c.len = ch.len;
  c.nvec = ch.len >> 2;
  c.vec = c.nvec > 0 &&
          !((reinterpret_cast<uintptr_t>(c.p) | reinterpret_cast<uintptr_t>(c.m) |
             reinterpret_cast<uintptr_t>(c.v)) & 15u) &&
          !(reinterpret_cast<uintptr_t>(c.g) & (sizeof(typename G::slot4) - 1)) &&
          !(c.p16 && (reinterpret_cast<uintptr_t>(c.p16) & 7u));
  return c;
}

// A trip of U slots per thread in registers.
template <int GD, int U>
struct Trip {
  typename Grad<GD>::slot4 g[U];
  f4 p[U], m[U], v[U];
};

// Issue a chunk's first trip of slot loads. Every thread issues the same
// loads whatever the chunk: indices clamped into the chunk, and for a chunk
// off the slot path loads from `spare` rounded down to 16 bytes (the tensor
// table: device allocations start on 256-byte boundaries, so that stays in
// the table's allocation; the values go unused), so that the waits for them
// stay exact.
template <int GD, int U, bool NT>
__device__ __forceinline__ void first_trip(const ChunkView<GD>& c, const void* spare_any, Trip<GD, U>& T) {
  using GS = typename Grad<GD>::slot4;
  const void* spare = reinterpret_cast<const void*>(reinterpret_cast<uintptr_t>(spare_any) & ~uintptr_t(15));
  const f4* lp = c.vec ? reinterpret_cast<const f4*>(c.p) : static_cast<const f4*>(spare);
  const f4* lm = c.vec ? reinterpret_cast<const f4*>(c.m) : static_cast<const f4*>(spare);
  const f4* lv = c.vec ? reinterpret_cast<const f4*>(c.v) : static_cast<const f4*>(spare);
  const GS* lg = c.vec ? reinterpret_cast<const GS*>(c.g) : static_cast<const GS*>(spare);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    int64_t i = (int64_t)threadIdx.x + (int64_t)u * kBlock;
    i = !c.vec ? 0 : (i < c.nvec ? i : c.nvec - 1);
    T.g[u] = ld<NT>(lg + i);
    T.p[u] = ld<NT>(lp + i);
    T.m[u] = ld<NT>(lm + i);
    T.v[u] = ld<NT>(lv + i);
  }
}

// Step a chunk whose first trip first_trip has loaded: the K2 slot loop (U
// slots per thread, each trip's loads issued before the previous trip's
// math), then the tail elements; element by element for a chunk off the slot
// path.
template <int GD, int PD, int U, bool NT, bool DRAIN>
__device__ __forceinline__ void chunk_steps(const ChunkView<GD>& c, Trip<GD, U>& T, const Sc& sc) {
  using G = Grad<GD>;
  using GS = typename G::slot4;
  const bool cast = c.p16 != nullptr;
  int64_t done = 0;
  if (c.vec) {
    f4* p4 = reinterpret_cast<f4*>(c.p);
    f4* m4 = reinterpret_cast<f4*>(c.m);
    f4* v4 = reinterpret_cast<f4*>(c.v);
    u2* o2 = reinterpret_cast<u2*>(c.p16);
    const GS* g4 = reinterpret_cast<const GS*>(c.g);
    for (int64_t i0 = threadIdx.x;;) {
      // Every slot's loads are taken in here, on every path: a slot past the
      // end (a clamped copy, dropped below) would otherwise leave its loads
      // pending into the next trip, whose first register writes would then
      // wait for this trip's stores too.
#pragma unroll
      for (int u = 0; u < U; ++u) asm volatile("" : "+v"(T.g[u]), "+v"(T.p[u]), "+v"(T.m[u]), "+v"(T.v[u]));
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = i0 + (int64_t)u * kBlock;
        if (i < c.nvec) {
          float gf[4];
          G::four(T.g[u], gf);
          f4 pp = T.p[u], mm = T.m[u], vv = T.v[u];
          adamw4(gf, pp, mm, vv, sc);
          st<NT>(p4 + i, pp);
          st<NT>(m4 + i, mm);
          st<NT>(v4 + i, vv);
          if (cast) st<NT>(o2 + i, pack4<PD>(pp));
        }
      }
      if constexpr (DRAIN) __builtin_amdgcn_s_waitcnt(0);  // as in k2_adamw_flat
      i0 += (int64_t)kBlock * U;
      if (i0 >= c.nvec) break;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int64_t i = i0 + (int64_t)u * kBlock;
        i = i < c.nvec ? i : c.nvec - 1;
        T.g[u] = ld<NT>(g4 + i);
        T.p[u] = ld<NT>(p4 + i);
        T.m[u] = ld<NT>(m4 + i);
        T.v[u] = ld<NT>(v4 + i);
      }
    }
    done = c.nvec << 2;
  }
  for (int64_t e = done + threadIdx.x; e < c.len; e += kBlock) {
    float pe = c.p[e], me = c.m[e], ve = c.v[e];
    adamw_elt(G::one(c.g[e]), pe, me, ve, sc);
    c.p[e] = pe; c.m[e] = me; c.v[e] = ve;
    if (cast) c.p16[e] = (uint16_t)f2h<PD>(pe);
  }
}

// K3: AdamW + cast over a chunk table. Block b steps chunks b, b + grid, ...
// Each chunk's records are read while the block works: the next chunk's
// record (a line of the table no block has read yet, so a trip to memory) is
// requested once this chunk's first slot loads and its group's scalars are
// in, and is consumed after this chunk's last trip.
template <int GD, int PD, int U, bool NT, bool DRAIN>
__global__ __launch_bounds__(kBlock) void k2_adamw_multi(const DsxTensorRef* __restrict__ tensors,
                                                         const DsxChunk* __restrict__ chunks, int64_t nchunks,
                                                         const DsxStepScalars* __restrict__ scalars) {
  if (((ConstScalars)(uintptr_t)scalars)->skip) return;  // the skip decision is global
  const int64_t stride = gridDim.x;  // in a register: the loop's asm barrier would reload it
  int64_t c = blockIdx.x;  // < nchunks: the grid is at most the chunk count
  DsxChunk ch = chunk_rec(chunks, c);
  for (;;) {
    const DsxTensorRef tr = tensor_rec(tensors, ch.tensor);
    const ChunkView<GD> cv = chunk_view<GD>(tr, ch);
    Trip<GD, U> T;
    first_trip<GD, U, NT>(cv, tensors, T);
    const Sc sc = scalars_rec(scalars, tr.group);
    asm volatile("" ::"s"(sc.nss) : "memory");  // the scalars are in before the next record is asked for
    const int64_t cn = c + stride;
    const DsxChunk chn = chunk_rec(chunks, cn < nchunks ? cn : c);
    chunk_steps<GD, PD, U, NT, DRAIN>(cv, T, sc);
    if (cn >= nchunks) break;
    c = cn;
    ch = chn;
  }
}

// K3 with K0's finalize folded in (the ragged form of k2_adamw_fold, after a
// K1 over the list launched with fold): every block reduces the partials in
// K0's order and decides the step with K0's code on the entry values, then
// steps its chunk with its group's scalars; the last block does no chunk
// work and writes the step records and the state's updated fields. One
// chunk per block (the small-list shape: the grid is the chunk count and the
// writer); 1 <= nparts <= kFoldMaxParts.
template <int GD, int PD, bool NT>
__global__ __launch_bounds__(kBlock) void k3_adamw_fold(const DsxTensorRef* __restrict__ tensors,
                                                        const DsxChunk* __restrict__ chunks, int64_t nchunks,
                                                        const double* __restrict__ partials, int32_t nparts,
                                                        DsxState* state, DsxScalerConfig scfg, DsxGroupsDev grp,
                                                        DsxStepScalars* __restrict__ out) {
  constexpr int U = 2;
  // The host launches nchunks + 1 blocks: one per chunk, then the writer (a
  // larger grid's extra blocks would return here).
  if ((int64_t)blockIdx.x > nchunks) return;
  if ((int64_t)blockIdx.x == nchunks) {
    double x = 0.0;
    for (int i = threadIdx.x; i < nparts; i += kBlock) x += partials[i];  // reduce_partials' order
    const double sumsq = block_sum_all(x);
    if (threadIdx.x == 0) {
      DsxState f = *state;
      f.clip_once = f.step_t2 & 1;  // K1 consumed the live flag into step_t2
      const Decision d = decide(sumsq, f, grp, false);
      for (int k = 0; k < grp.ngroups; ++k) out[k] = record(d, f, grp, k, sumsq);
      advance(d, f, scfg);
      state->scale = f.scale;
      state->good_steps = f.good_steps;
      state->hyst_left = f.hyst_left;
      state->t = f.t;
      state->iter = f.iter;
      state->overflow_count = f.overflow_count;
      state->error = f.error;
      state->last_skip = f.last_skip;
      state->last_norm = f.last_norm;
      state->clip_once = 0;
    }
    return;
  }
  // As in k2_adamw_fold: the entry values, the partials' loads and this
  // block's chunk's first trip of slot loads are all issued before any is
  // used (an unaligned chunk's slot loads read the tensor table instead, and
  // are not used: every path issues the same loads).
  int32_t t2 = state->step_t2;
  float scale0 = state->step_scale, coef1 = state->clip_once_coef;
  double pv[kFoldParts];
#pragma unroll
  for (int j = 0; j < kFoldParts; ++j) {
    const int i = threadIdx.x + j * kBlock;
    const double x = partials[i < nparts ? i : nparts - 1];
    pv[j] = i < nparts ? x : 0.0;
  }
  const DsxChunk ch = chunk_rec(chunks, blockIdx.x);  // < nchunks: nchunks slot blocks and the writer
  const DsxTensorRef tr = tensor_rec(tensors, ch.tensor);
  const ChunkView<GD> cv = chunk_view<GD>(tr, ch);
  Trip<GD, U> T;
  first_trip<GD, U, NT>(cv, tensors, T);
  asm volatile("" ::: "memory");  // the slot loads issue here
  asm volatile("" : "+v"(t2), "+v"(scale0), "+v"(coef1));
  DsxState s = {};
  s.scale = scale0;
  t2 = __builtin_amdgcn_readfirstlane(t2);
  s.t = t2 >> 1;
  s.clip_once = t2 & 1;
  s.clip_once_coef = coef1;
  double bc1 = 1.0, bc2s = 1.0;
  if (tr.group < grp.ngroups) bc_of(grp, tr.group, s.t + 1, bc1, bc2s);
  asm volatile("" : "+v"(pv[0]), "+v"(pv[1]));
  double x = 0.0;
#pragma unroll
  for (int j = 0; j < kFoldParts; ++j) x += pv[j];  // reduce_partials' order
  const double sumsq = block_sum_all(x);
  const Decision d = decide(sumsq, s, grp, false);
  if (d.skip || tr.group >= d.ng) return;
  const Sc sc = uniform_sc(load_sc(record_bc(d, s, grp, tr.group, sumsq, bc1, bc2s)));
  chunk_steps<GD, PD, U, NT, false>(cv, T, sc);
}

// ---- host-side dispatch ----------------------------------------------------------

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

template <int GD>
void launch_k1(const void* g, int64_t n, const DsxState* st, double* partials, int nparts, DsxState* fold,
               hipStream_t s) {
  if (g_tune.nontemporal)
    hipLaunchKernelGGL((k1_unscale_norm<GD, 4, true>), dim3(nparts), dim3(kBlock), 0, s, g, n, st, partials, fold);
  else
    hipLaunchKernelGGL((k1_unscale_norm<GD, 4, false>), dim3(nparts), dim3(kBlock), 0, s, g, n, st, partials, fold);
}

template <int GD, int PD, int U, bool NT, bool DRAIN>
void k2_launch_one(bool probe, dim3 grid, hipStream_t s, float* p, float* m, float* v, uint16_t* o, const void* g,
                   int64_t n, const DsxStepScalars* sc) {
  if constexpr (GD == PD) {  // the probe is built for 16-bit training only
    if (probe) {
      hipLaunchKernelGGL((k2_traffic_probe<GD, PD, U, NT, DRAIN>), grid, dim3(kBlock), 0, s, p, m, v, o, g, n, sc);
      return;
    }
  }
  hipLaunchKernelGGL((k2_adamw_flat<GD, PD, U, NT, DRAIN>), grid, dim3(kBlock), 0, s, p, m, v, o, g, n, sc);
}

template <int GD, int PD, int U>
void launch_k2_u(float* p, float* m, float* v, void* p16, const void* g, int64_t n, const DsxStepScalars* sc,
                 hipStream_t s, bool probe) {
  const int64_t slots = n >> 2;
  int64_t blocks = ceil_div(slots > 0 ? slots : 1, (int64_t)kBlock * U);  // one trip each
  const bool large = n >= kK2LargeN;
  const int eighths = g_tune.k2_cu_eighths ? g_tune.k2_cu_eighths : (large ? 7 : 8);
  const bool drain = g_tune.k2_drain >= 0 ? g_tune.k2_drain != 0 : large;
  const int64_t cus = cu_count();
  int64_t cap;
  if (g_tune.k2_blocks_per_cu > 0)
    cap = cus * g_tune.k2_blocks_per_cu * eighths / 8;
  else if (!large && blocks <= cus * kK2OneTripPerCu)
    cap = blocks;
  else
    cap = cus * eighths / 8;
  if (cap < 1) cap = 1;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  uint16_t* o = static_cast<uint16_t*>(p16);
  const dim3 grid((unsigned)blocks);
  if (g_tune.nontemporal) {
    if (drain)
      k2_launch_one<GD, PD, U, true, true>(probe, grid, s, p, m, v, o, g, n, sc);
    else
      k2_launch_one<GD, PD, U, true, false>(probe, grid, s, p, m, v, o, g, n, sc);
  } else {
    if (drain)
      k2_launch_one<GD, PD, U, false, true>(probe, grid, s, p, m, v, o, g, n, sc);
    else
      k2_launch_one<GD, PD, U, false, false>(probe, grid, s, p, m, v, o, g, n, sc);
  }
}

template <int GD, int PD>
void launch_k2(float* p, float* m, float* v, void* p16, const void* g, int64_t n, const DsxStepScalars* sc,
               hipStream_t s, bool probe) {
  const int unroll = g_tune.k2_unroll ? g_tune.k2_unroll : (n >= kK2LargeN ? 4 : 2);
  switch (unroll) {
    case 2: launch_k2_u<GD, PD, 2>(p, m, v, p16, g, n, sc, s, probe); break;
    case 8: launch_k2_u<GD, PD, 8>(p, m, v, p16, g, n, sc, s, probe); break;
    default: launch_k2_u<GD, PD, 4>(p, m, v, p16, g, n, sc, s, probe); break;
  }
}

int check_flat(const float* master, const float* m, const float* v, const void* p16, int pdt, const void* g,
               int gdt, int64_t n) {
  if (n < 0) return fail(DSX_EINVAL, "n must be >= 0 (got %lld)", (long long)n);
  if (!is_grad_dtype(gdt)) return fail(DSX_EINVAL, "grad dtype must be DSX_F16, DSX_BF16 or DSX_F32 (got %d)", gdt);
  if (p16 && !is16(pdt)) return fail(DSX_EINVAL, "param16 dtype must be DSX_F16 or DSX_BF16 (got %d)", pdt);
  if (n == 0) return DSX_OK;
  if (!master || !m || !v || !g) return fail(DSX_EINVAL, "null master/exp_avg/exp_avg_sq/grad pointer");
  if (!aligned16(master) || !aligned16(m) || !aligned16(v) || !aligned16(g) || (p16 && !aligned16(p16)))
    return fail(DSX_EINVAL, "flat buffers must be 16-byte aligned");
  return DSX_OK;
}

int check_hyper(const DsxAdamwHyper& h) {
  // Same admissible ranges as torch.optim.Adam's constructor (torch/optim/adam.py).
  if (!(h.lr >= 0.0)) return fail(DSX_EINVAL, "Invalid learning rate: %g", h.lr);
  if (!(h.eps >= 0.0)) return fail(DSX_EINVAL, "Invalid epsilon value: %g", h.eps);
  if (!(h.beta1 >= 0.0 && h.beta1 < 1.0)) return fail(DSX_EINVAL, "Invalid beta parameter at index 0: %g", h.beta1);
  if (!(h.beta2 >= 0.0 && h.beta2 < 1.0)) return fail(DSX_EINVAL, "Invalid beta parameter at index 1: %g", h.beta2);
  if (!(h.weight_decay >= 0.0)) return fail(DSX_EINVAL, "Invalid weight_decay value: %g", h.weight_decay);
  if (!(h.clip_eps >= 0.0)) return fail(DSX_EINVAL, "Invalid clip_eps: %g", h.clip_eps);
  if (h.max_grad_norm != h.max_grad_norm) return fail(DSX_EINVAL, "max_grad_norm is NaN");
  return DSX_OK;
}

int check_scaler(const DsxScalerConfig& c) {
  if (c.mode < DSX_SCALE_NONE || c.mode > DSX_SCALE_DYNAMIC) return fail(DSX_EINVAL, "bad scaler mode %d", c.mode);
  if (c.mode == DSX_SCALE_DYNAMIC) {
    if (c.window < 1) return fail(DSX_EINVAL, "loss_scale_window must be >= 1 (got %d)", c.window);
    if (c.hysteresis < 1) return fail(DSX_EINVAL, "hysteresis must be >= 1 (got %d)", c.hysteresis);
    if (!(c.min_scale > 0.0f)) return fail(DSX_EINVAL, "min_loss_scale must be > 0 (got %g)", c.min_scale);
    if (!(c.growth_factor > 1.0f)) return fail(DSX_EINVAL, "growth_factor must be > 1 (got %g)", c.growth_factor);
    if (!(c.backoff_factor > 0.0f && c.backoff_factor < 1.0f))
      return fail(DSX_EINVAL, "backoff_factor must be in (0, 1) (got %g)", c.backoff_factor);
  }
  return DSX_OK;
}

int check_parts(const double* partials, int32_t nparts) {
  if (nparts < 1 || nparts > DSX_MAX_PARTIALS)
    return fail(DSX_EINVAL, "nparts must be in [1, %d] (got %d)", DSX_MAX_PARTIALS, nparts);
  if (!partials) return fail(DSX_EINVAL, "null partials");
  return DSX_OK;
}

int do_unscale_norm(const void* g, int gdt, int64_t n, const DsxState* st, double* partials, int32_t nparts,
                    hipStream_t s, DsxState* fold = nullptr) {
  switch (gdt) {
    case DSX_BF16: launch_k1<DSX_BF16>(g, n, st, partials, nparts, fold, s); break;
    case DSX_F16: launch_k1<DSX_F16>(g, n, st, partials, nparts, fold, s); break;
    default: launch_k1<DSX_F32>(g, n, st, partials, nparts, fold, s); break;
  }
  return launch_status("dsx_unscale_norm");
}

int do_finalize(const double* partials, int32_t nparts, DsxState* st, const DsxScalerConfig& sc,
                const DsxGroupsDev& grp, DsxStepScalars* out, hipStream_t s) {
  hipLaunchKernelGGL(k0_finalize, dim3(1), dim3(kBlock), 0, s, partials, nparts, st, sc, grp, out);
  return launch_status("dsx_finalize");
}

DsxGroupsDev one_group(const DsxAdamwHyper& hp, const double* bc, int32_t bc_len) {
  DsxGroupsDev g = {};
  g.hyper[0] = hp;
  g.bc_table[0] = bc;
  g.t_offset[0] = 0;
  g.ngroups = 1;
  g.bc_len = bc_len;
  return g;
}

template <int GD>
void k2_by_param(int pd, float* p, float* m, float* v, void* p16, const void* g, int64_t n,
                 const DsxStepScalars* sc, hipStream_t s, bool probe = false) {
  if (pd == DSX_BF16) launch_k2<GD, DSX_BF16>(p, m, v, p16, g, n, sc, s, probe);
  else launch_k2<GD, DSX_F16>(p, m, v, p16, g, n, sc, s, probe);
}

// K2 (or its traffic probe) over n elements as consecutive launches of at
// most ~g_tune.k2_chunk_elems elements each (equal parts, multiples of 1024
// elements, so every part stays 16-byte aligned and only the last has a
// tail). Each part takes the launch shape of its own size.
void k2_dispatch(float* p, float* m, float* v, void* p16, int pdt, const void* g, int gdt, int64_t n,
                 const DsxStepScalars* sc, hipStream_t s, bool probe) {
  const int pd = p16 ? pdt : DSX_F16;  // pd only selects the cast when p16 != NULL
  const int64_t want = g_tune.k2_chunk_elems;
  int64_t part = n;
  if (want > 0 && n > want) part = ceil_div(ceil_div(n, ceil_div(n, want)), 1024) * 1024;
  const int64_t gsz = gdt == DSX_F32 ? 4 : 2;
  for (int64_t a = 0; a < n; a += part) {
    const int64_t len = n - a < part ? n - a : part;
    float* pa = p + a;
    float* ma = m + a;
    float* va = v + a;
    void* oa = p16 ? static_cast<void*>(static_cast<uint16_t*>(p16) + a) : nullptr;
    const void* ga = static_cast<const char*>(g) + a * gsz;
    switch (gdt) {
      case DSX_BF16: k2_by_param<DSX_BF16>(pd, pa, ma, va, oa, ga, len, sc, s, probe); break;
      case DSX_F16: k2_by_param<DSX_F16>(pd, pa, ma, va, oa, ga, len, sc, s, probe); break;
      default: k2_by_param<DSX_F32>(pd, pa, ma, va, oa, ga, len, sc, s, probe); break;
    }
  }
}

int do_adamw_flat(float* p, float* m, float* v, void* p16, int pdt, const void* g, int gdt, int64_t n,
                  const DsxStepScalars* sc, hipStream_t s) {
  if (n == 0) return DSX_OK;
  k2_dispatch(p, m, v, p16, pdt, g, gdt, n, sc, s, false);
  return launch_status("dsx_adamw_flat");
}

// Where the folded K2 takes the group block from: a host block passed as a
// kernel argument (checked on the host), or a block in device memory with
// max_groups record slots (checked in the kernel; the graph form).
struct FoldGroups {
  const DsxGroupsDev* host;
  const DsxGroupsDev* dev;
  int32_t max_groups;
};

// The folded K2 over one group's range: the one-trip grid of K2 (2 slots per
// thread, at most kK2OneTripPerCu blocks per CU; the kernel strides over what
// one trip does not cover), plus the writer's block.
template <int GD, int PD, bool NT>
void launch_k2_fold_nt(dim3 grid, float* p, float* m, float* v, uint16_t* o, const void* g, int64_t n,
                       const double* partials, int32_t nparts, DsxState* state, const DsxScalerConfig& scfg,
                       const FoldGroups& fg, int group, int32_t w, DsxStepScalars* out, hipStream_t s) {
  constexpr int U = 2;
  if (fg.dev)
    hipLaunchKernelGGL((k2_adamw_fold<GD, PD, U, NT, const DsxGroupsDev*>), grid, dim3(kBlock), 0, s, p, m, v, o, g,
                       n, partials, nparts, state, scfg, fg.dev, fg.max_groups, group, w, out);
  else
    hipLaunchKernelGGL((k2_adamw_fold<GD, PD, U, NT, DsxGroupsDev>), grid, dim3(kBlock), 0, s, p, m, v, o, g, n,
                       partials, nparts, state, scfg, *fg.host, fg.max_groups, group, w, out);
}

template <int GD, int PD>
void launch_k2_fold(float* p, float* m, float* v, void* p16, const void* g, int64_t n, const double* partials,
                    int32_t nparts, DsxState* state, const DsxScalerConfig& scfg, const FoldGroups& fg,
                    int group, bool writer, DsxStepScalars* out, hipStream_t s, int64_t blocks_per_cu) {
  const int64_t slots = n >> 2;
  int64_t blocks = ceil_div(slots > 0 ? slots : 1, (int64_t)kBlock * 2);
  const int64_t cap = (int64_t)cu_count() * blocks_per_cu;
  if (blocks > cap) blocks = cap;
  if (writer) blocks += 1;  // the block that writes the records and the state
  uint16_t* o = static_cast<uint16_t*>(p16);
  const dim3 grid((unsigned)blocks);
  const int32_t w = writer ? 1 : 0;
  if (g_tune.nontemporal)
    launch_k2_fold_nt<GD, PD, true>(grid, p, m, v, o, g, n, partials, nparts, state, scfg, fg, group, w, out, s);
  else
    launch_k2_fold_nt<GD, PD, false>(grid, p, m, v, o, g, n, partials, nparts, state, scfg, fg, group, w, out, s);
}

template <int GD>
void k2_fold_by_param(int pd, float* p, float* m, float* v, void* p16, const void* g, int64_t n,
                      const double* partials, int32_t nparts, DsxState* state, const DsxScalerConfig& scfg,
                      const FoldGroups& fg, int group, bool writer, DsxStepScalars* out, hipStream_t s,
                      int64_t bpc) {
  if (pd == DSX_BF16)
    launch_k2_fold<GD, DSX_BF16>(p, m, v, p16, g, n, partials, nparts, state, scfg, fg, group, writer, out, s, bpc);
  else
    launch_k2_fold<GD, DSX_F16>(p, m, v, p16, g, n, partials, nparts, state, scfg, fg, group, writer, out, s, bpc);
}

bool fold_applies(int64_t n, int32_t nparts) {
  return g_tune.fold_max_elems > 0 && n >= 4 && n <= g_tune.fold_max_elems && nparts <= kFoldMaxParts;
}

// Above the fold's bound, K0 is folded into the first of K2's parts alone,
// launched one block per CU (so that few blocks pay the partials' reduction),
// and the other parts read the records that launch's writer block wrote.
// Like the whole fold, it needs n >= 4 (a bound of 1 to 3 set through
// dsx_set_tuning_fold would otherwise send 2 or 3 elements to it).
bool fold_first_applies(int64_t n, int32_t nparts) {
  return g_tune.fold_max_elems > 0 && n >= 4 && n > g_tune.fold_max_elems && nparts <= kFoldMaxParts;
}

// The length of K2's first part over n elements (k2_dispatch's split).
int64_t k2_first_part(int64_t n) {
  const int64_t want = g_tune.k2_chunk_elems;
  if (want <= 0 || n <= want) return n;
  return ceil_div(ceil_div(n, ceil_div(n, want)), 1024) * 1024;
}

// The folded K2 over n elements: K2's one-trip grid (at most
// kK2OneTripPerCu blocks per CU), or at most bpc blocks per CU.
int do_adamw_fold(float* p, float* m, float* v, void* p16, int pdt, const void* g, int gdt, int64_t n,
                  const double* partials, int32_t nparts, DsxState* state, const DsxScalerConfig& scfg,
                  const FoldGroups& fg, int group, bool writer, DsxStepScalars* out, hipStream_t s,
                  int64_t bpc = kK2OneTripPerCu) {
  const int pd = p16 ? pdt : DSX_F16;
  switch (gdt) {
    case DSX_BF16:
      k2_fold_by_param<DSX_BF16>(pd, p, m, v, p16, g, n, partials, nparts, state, scfg, fg, group, writer, out, s,
                                 bpc);
      break;
    case DSX_F16:
      k2_fold_by_param<DSX_F16>(pd, p, m, v, p16, g, n, partials, nparts, state, scfg, fg, group, writer, out, s,
                                bpc);
      break;
    default:
      k2_fold_by_param<DSX_F32>(pd, p, m, v, p16, g, n, partials, nparts, state, scfg, fg, group, writer, out, s,
                                bpc);
      break;
  }
  return launch_status("dsx_adamw_flat (finalize folded in)");
}

template <int GD, int PD, int U>
void launch_k3_u(bool drain, dim3 grid, const DsxTensorRef* t, const DsxChunk* c, int64_t nc,
                 const DsxStepScalars* sc, hipStream_t s) {
  if (g_tune.k3_nontemporal) {
    if (drain)
      hipLaunchKernelGGL((k2_adamw_multi<GD, PD, U, true, true>), grid, dim3(kBlock), 0, s, t, c, nc, sc);
    else
      hipLaunchKernelGGL((k2_adamw_multi<GD, PD, U, true, false>), grid, dim3(kBlock), 0, s, t, c, nc, sc);
  } else {
    if (drain)
      hipLaunchKernelGGL((k2_adamw_multi<GD, PD, U, false, true>), grid, dim3(kBlock), 0, s, t, c, nc, sc);
    else
      hipLaunchKernelGGL((k2_adamw_multi<GD, PD, U, false, false>), grid, dim3(kBlock), 0, s, t, c, nc, sc);
  }
}

template <int GD, int PD>
void launch_k3_p(int unroll, bool drain, dim3 grid, const DsxTensorRef* t, const DsxChunk* c, int64_t nc,
                 const DsxStepScalars* sc, hipStream_t s) {
  switch (unroll) {
    case 1: launch_k3_u<GD, PD, 1>(drain, grid, t, c, nc, sc, s); break;
    case 4: launch_k3_u<GD, PD, 4>(drain, grid, t, c, nc, sc, s); break;
    default: launch_k3_u<GD, PD, 2>(drain, grid, t, c, nc, sc, s); break;
  }
}

template <int GD>
void launch_k3(int pd, int unroll, bool drain, dim3 grid, const DsxTensorRef* t, const DsxChunk* c, int64_t nc,
               const DsxStepScalars* sc, hipStream_t s) {
  if (pd == DSX_BF16) launch_k3_p<GD, DSX_BF16>(unroll, drain, grid, t, c, nc, sc, s);
  else launch_k3_p<GD, DSX_F16>(unroll, drain, grid, t, c, nc, sc, s);
}

int norm_kind(double p, int* kind) {
  if (!(p > 0.0)) return fail(DSX_EINVAL, "norm_type must be > 0 (finite or inf), got %g", p);
  *kind = __builtin_isinf(p) ? kNormMax : p == 2.0 ? kNormSq : p == 1.0 ? kNormAbs : kNormPow;
  return DSX_OK;
}

template <int GD, int K>
void launch_norm_k(bool multi, const void* g, int64_t n, const DsxTensorRef* t, const DsxChunk* c, int64_t nc,
                   const DsxState* st, double p, double* partials, int nparts, hipStream_t s) {
  const dim3 grid((unsigned)nparts), blk(kBlock);
  if (multi)
    hipLaunchKernelGGL((k1_norm_multi<GD, K>), grid, blk, 0, s, t, c, nc, st, p, partials);
  else
    hipLaunchKernelGGL((k1_norm<GD, K>), grid, blk, 0, s, g, n, st, p, partials);
}

template <int GD>
void launch_norm(int kind, bool multi, const void* g, int64_t n, const DsxTensorRef* t, const DsxChunk* c,
                 int64_t nc, const DsxState* st, double p, double* partials, int nparts, hipStream_t s) {
  switch (kind) {
    case kNormSq: launch_norm_k<GD, kNormSq>(multi, g, n, t, c, nc, st, p, partials, nparts, s); break;
    case kNormAbs: launch_norm_k<GD, kNormAbs>(multi, g, n, t, c, nc, st, p, partials, nparts, s); break;
    case kNormMax: launch_norm_k<GD, kNormMax>(multi, g, n, t, c, nc, st, p, partials, nparts, s); break;
    default: launch_norm_k<GD, kNormPow>(multi, g, n, t, c, nc, st, p, partials, nparts, s); break;
  }
}

int do_norm(int gdt, int kind, bool multi, const void* g, int64_t n, const DsxTensorRef* t, const DsxChunk* c,
            int64_t nc, const DsxState* st, double p, double* partials, int nparts, hipStream_t s) {
  switch (gdt) {
    case DSX_BF16: launch_norm<DSX_BF16>(kind, multi, g, n, t, c, nc, st, p, partials, nparts, s); break;
    case DSX_F16: launch_norm<DSX_F16>(kind, multi, g, n, t, c, nc, st, p, partials, nparts, s); break;
    default: launch_norm<DSX_F32>(kind, multi, g, n, t, c, nc, st, p, partials, nparts, s); break;
  }
  return launch_status(multi ? "dsx_norm_partials_multi" : "dsx_norm_partials");
}

// Argument checks of the flat step, shared by dsx_zero_step_flat and its
// no-allocation variant (everything but the scratch buffers).
int check_zero_step(const float* master, const float* m, const float* v, const void* p16, int pdt, const void* g,
                    int gdt, int64_t n, const DsxState* state, const DsxScalerConfig& scaler,
                    const DsxAdamwHyper& hyper, const double* bc_table, int32_t bc_len) {
  int rc = check_flat(master, m, v, p16, pdt, g, gdt, n);
  if (!rc) rc = check_scaler(scaler);
  if (!rc) rc = check_hyper(hyper);
  if (rc) return rc;
  if (!state) return fail(DSX_EINVAL, "null state");
  if (bc_len < 0 || (bc_len > 0 && !bc_table)) return fail(DSX_EINVAL, "bad bias-correction table");
  return DSX_OK;
}

int zero_step_flat(float* master, float* m, float* v, void* p16, int pdt, const void* g, int gdt, int64_t n,
                   DsxState* state, const DsxScalerConfig& scaler, const DsxAdamwHyper& hyper,
                   const double* bc_table, int32_t bc_len, double* partials, int32_t nparts, DsxStepScalars* out,
                   hipStream_t s) {
  const DsxGroupsDev grp = one_group(hyper, bc_table, bc_len);
  if (fold_applies(n, nparts)) {
    int rc = do_unscale_norm(g, gdt, n, state, partials, nparts, s, state);
    if (!rc) rc = do_adamw_fold(master, m, v, p16, pdt, g, gdt, n, partials, nparts, state, scaler,
                                FoldGroups{&grp, nullptr, 1}, 0, true, out, s);
    return rc;
  }
  if (fold_first_applies(n, nparts)) {
    const int64_t a = k2_first_part(n);
    int rc = do_unscale_norm(g, gdt, n, state, partials, nparts, s, state);
    if (!rc) rc = do_adamw_fold(master, m, v, p16, pdt, g, gdt, a, partials, nparts, state, scaler,
                                FoldGroups{&grp, nullptr, 1}, 0, true, out, s, 1);
    if (!rc && a < n) {
      void* p16a = p16 ? static_cast<void*>(static_cast<uint16_t*>(p16) + a) : nullptr;
      const void* ga = static_cast<const char*>(g) + a * (gdt == DSX_F32 ? 4 : 2);
      rc = do_adamw_flat(master + a, m + a, v + a, p16a, pdt, ga, gdt, n - a, out, s);
    }
    return rc;
  }
  int rc = do_unscale_norm(g, gdt, n, state, partials, nparts, s);
  if (!rc) rc = do_finalize(partials, nparts, state, scaler, grp, out, s);
  if (!rc) rc = do_adamw_flat(master, m, v, p16, pdt, g, gdt, n, out, s);
  return rc;
}

// The address of `scratch` on the current device, resolved once per device
// with hipGetSymbolAddress (each GPU holds its own copy at its own address)
// and checked to be the device the stream runs on.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_ptr[kMaxDevices];

int noalloc_scratch(hipStream_t s, unsigned char** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail((int)e, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(DSX_EINVAL, "device %d out of range [0, %d)", dev, kMaxDevices);
  hipDevice_t sdev = -1;
  e = hipStreamGetDevice(s, &sdev);
  if (e != hipSuccess) return fail((int)e, "hipStreamGetDevice failed: %s", hipGetErrorString(e));
  if ((int)sdev != dev)
    return fail(DSX_EINVAL, "the stream belongs to device %d but device %d is current", (int)sdev, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(e != hipSuccess ? (int)e : DSX_EINVAL, "hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<unsigned char*>(p);
  }
  *out = g_scratch_ptr[dev];
  return DSX_OK;
}

template <int GD>
void launch_k1_multi(bool wave, dim3 grid, const DsxTensorRef* tensors, const DsxChunk* chunks, int64_t nchunks,
                     const DsxState* state, double* partials, DsxState* fold, hipStream_t s) {
  if (wave)
    hipLaunchKernelGGL((k1_unscale_norm_multi<GD, true>), grid, dim3(kBlock), 0, s, tensors, chunks, nchunks,
                       state, partials, fold);
  else
    hipLaunchKernelGGL((k1_unscale_norm_multi<GD, false>), grid, dim3(kBlock), 0, s, tensors, chunks, nchunks,
                       state, partials, fold);
}

// K1 over a chunk table. Each wave takes its own chunks when the table has
// at most 16 chunks per block (kK1WaveChunksPerPart), one block per chunk
// otherwise: decided from the chunk and partial counts alone, so that every
// entry point over the same table and partials takes the same shape and sums
// in the same order. The tables the library builds have chunks of 2048 to
// 16384 elements up to that count, 65536 beyond it; per launch on MI355X
// (one process, alternated): 4096-element chunks over 2.1e7 elements 12.7 ->
// 9.3 us and over 8.6e7 49.7 -> 28.7 us, 16384-element chunks over 1.2e8
// 39.1 -> 39.5 us, 65536-element chunks over 2.9e9 and 8.3e9 elements 2-4%
// slower one wave per chunk.
constexpr int64_t kK1WaveChunksPerPart = 16;
int do_unscale_norm_multi(const DsxTensorRef* tensors, const DsxChunk* chunks, int64_t nchunks, int gdt,
                          const DsxState* state, double* partials, int32_t nparts, hipStream_t s, DsxState* fold) {
  const dim3 grid(nparts);
  const bool wave = nchunks <= kK1WaveChunksPerPart * nparts;
  switch (gdt) {
    case DSX_BF16: launch_k1_multi<DSX_BF16>(wave, grid, tensors, chunks, nchunks, state, partials, fold, s); break;
    case DSX_F16: launch_k1_multi<DSX_F16>(wave, grid, tensors, chunks, nchunks, state, partials, fold, s); break;
    default: launch_k1_multi<DSX_F32>(wave, grid, tensors, chunks, nchunks, state, partials, fold, s); break;
  }
  return launch_status("dsx_unscale_norm_multi");
}

int do_adamw_multi(const DsxTensorRef* tensors, const DsxChunk* chunks, int64_t nchunks, int param_dtype,
                   int grad_dtype, const DsxStepScalars* scalars, hipStream_t s) {
  if (nchunks == 0) return DSX_OK;
  // Chunks are handed out statically (block b takes b, b + grid, ...). The
  // default shape, from sweeps on MI355X over ragged lists of 1e6 to 8.3e9
  // elements, two slots per trip throughout: up to 20 chunks per CU, one
  // chunk per block (all of a small list in flight at once: 1-11% faster
  // from 2 Mi to 16 Mi elements in 4096-element chunks, 2.5% slower at 30
  // chunks per CU); up to 256 chunks per
  // CU, one block per CU walking the list as one front (like K2's
  // grid-stride); from 256 chunks per CU on, a grid of about four chunks per
  // block, far more blocks than the CUs hold at once, with K2's drain, is
  // 4-5% faster (the blocks start as others finish). Five chunks per block
  // beat four by 0.5-0.7% over freshly allocated lists of 321 and 496 chunks
  // per CU, but lost by 0.6% in a process that had allocated and freed other
  // large buffers first (the same 496-chunk list, alternated), so four stay.
  const int64_t cus = cu_count();
  int64_t bpc = g_tune.k3_blocks_per_cu;
  int unroll = g_tune.k3_unroll;
  bool drain = g_tune.k3_drain > 0;
  if (bpc == 0) {
    const int64_t per_cu = nchunks / cus;
    const bool many = per_cu >= 256;
    if (nchunks <= kK3OneChunkPerCu * cus)
      bpc = ceil_div(nchunks, cus);  // one chunk per block
    else
      bpc = many ? per_cu / 4 : 1;
    unroll = 2;
    drain = g_tune.k3_drain >= 0 ? g_tune.k3_drain > 0 : many;
  }
  int64_t blocks = cus * bpc;
  if (blocks > nchunks) blocks = nchunks;
  // Blocks take chunks grid-stride, so any grid covers the table; keep it
  // within HIP's 2^32 work-items per grid dimension.
  if (blocks > kMaxGridBlocks) blocks = kMaxGridBlocks;
  const dim3 grid((unsigned)blocks);
  switch (grad_dtype) {
    case DSX_BF16: launch_k3<DSX_BF16>(param_dtype, unroll, drain, grid, tensors, chunks, nchunks, scalars, s); break;
    case DSX_F16: launch_k3<DSX_F16>(param_dtype, unroll, drain, grid, tensors, chunks, nchunks, scalars, s); break;
    default: launch_k3<DSX_F32>(param_dtype, unroll, drain, grid, tensors, chunks, nchunks, scalars, s); break;
  }
  return launch_status("dsx_adamw_multi");
}

template <int GD>
void launch_k3_fold(int pd, dim3 grid, const DsxTensorRef* t, const DsxChunk* c, int64_t nc, const double* partials,
                    int32_t nparts, DsxState* state, const DsxScalerConfig& scfg, const DsxGroupsDev& grp,
                    DsxStepScalars* out, hipStream_t s) {
  const bool nt = g_tune.k3_nontemporal != 0;
  if (pd == DSX_BF16) {
    if (nt)
      hipLaunchKernelGGL((k3_adamw_fold<GD, DSX_BF16, true>), grid, dim3(kBlock), 0, s, t, c, nc, partials, nparts,
                         state, scfg, grp, out);
    else
      hipLaunchKernelGGL((k3_adamw_fold<GD, DSX_BF16, false>), grid, dim3(kBlock), 0, s, t, c, nc, partials, nparts,
                         state, scfg, grp, out);
  } else {
    if (nt)
      hipLaunchKernelGGL((k3_adamw_fold<GD, DSX_F16, true>), grid, dim3(kBlock), 0, s, t, c, nc, partials, nparts,
                         state, scfg, grp, out);
    else
      hipLaunchKernelGGL((k3_adamw_fold<GD, DSX_F16, false>), grid, dim3(kBlock), 0, s, t, c, nc, partials, nparts,
                         state, scfg, grp, out);
  }
}

// The flat plan's own checks (everything but the group block).
int check_plan(const DsxFlatPlan& P) {
  int rc = check_flat(P.master, P.exp_avg, P.exp_avg_sq, P.param16, P.param_dtype, P.grad, P.grad_dtype, P.n);
  if (!rc) rc = check_parts(P.partials, P.nparts);
  if (!rc) rc = check_scaler(P.scaler);
  if (rc) return rc;
  if (!P.state || !P.out) return fail(DSX_EINVAL, "null state or scalars");
  if (P.ngroups < 1 || P.ngroups > DSX_MAX_GROUPS)
    return fail(DSX_EINVAL, "ngroups must be in [1, %d] (got %d)", DSX_MAX_GROUPS, P.ngroups);
  int64_t prev = 0;
  for (int k = 0; k < P.ngroups; ++k) {
    const int64_t end = P.group_end[k];
    const bool last = k == P.ngroups - 1;
    if (end < prev || end > P.n || (last ? end != P.n : (end & 7) != 0))
      return fail(DSX_EINVAL, "group_end[%d] = %lld: boundaries must be nondecreasing multiples of 8 ending at n",
                  k, (long long)end);
    prev = end;
  }
  return DSX_OK;
}

// The step of a checked plan: two launches (K1, then each nonempty group's K2
// with the finalize folded in, the first of them writing the state) where
// the fold applies, else three (K1, K0, each nonempty group's K2). The group
// block is the host's G (a kernel argument) or, when G is NULL, the block at
// the device address Gdev (read by the kernels: the graph form).
int plan_launches(const DsxFlatPlan& P, const DsxGroupsDev* G, const DsxGroupsDev* Gdev, hipStream_t s) {
  bool fold = fold_applies(P.n, P.nparts);
  bool first = !fold && fold_first_applies(P.n, P.nparts);  // fold K0 into the first part alone
  int64_t prev = 0;
  for (int k = 0; (fold || first) && k < P.ngroups; ++k) {
    const int64_t len = P.group_end[k] - prev;
    prev = P.group_end[k];
    if (len > 0 && len < 4) fold = first = false;  // the folded K2 takes at least one 4-element slot
  }
  int rc = do_unscale_norm(P.grad, P.grad_dtype, P.n, P.state, P.partials, P.nparts, s,
                           fold || first ? P.state : nullptr);
  if (!rc && !fold && !first) {
    if (G) {
      rc = do_finalize(P.partials, P.nparts, P.state, P.scaler, *G, P.out, s);
    } else {
      hipLaunchKernelGGL(k0_finalize_dev, dim3(1), dim3(kBlock), 0, s, P.partials, P.nparts, P.state, P.scaler, Gdev,
                         P.ngroups, P.out);
      rc = launch_status("dsx_finalize_dev");
    }
  }
  const FoldGroups fg{G, Gdev, P.ngroups};
  const int64_t gsz = P.grad_dtype == DSX_F32 ? 4 : 2;
  bool writer = true;
  prev = 0;
  for (int k = 0; !rc && k < P.ngroups; ++k) {
    const int64_t a = prev, b = P.group_end[k];
    prev = b;
    if (b == a) continue;
    void* p16 = P.param16 ? static_cast<void*>(static_cast<uint16_t*>(P.param16) + a) : nullptr;
    const void* ga = static_cast<const char*>(P.grad) + a * gsz;
    if (fold) {
      rc = do_adamw_fold(P.master + a, P.exp_avg + a, P.exp_avg_sq + a, p16, P.param_dtype, ga, P.grad_dtype, b - a,
                         P.partials, P.nparts, P.state, P.scaler, fg, k, writer, P.out, s);
    } else if (first && writer) {
      // The step's first part decides and writes the records; the rest of
      // this group and the other groups read them.
      const int64_t c = k2_first_part(b - a);
      rc = do_adamw_fold(P.master + a, P.exp_avg + a, P.exp_avg_sq + a, p16, P.param_dtype, ga, P.grad_dtype, c,
                         P.partials, P.nparts, P.state, P.scaler, fg, k, true, P.out, s, 1);
      if (!rc && c < b - a) {
        void* p16c = p16 ? static_cast<void*>(static_cast<uint16_t*>(p16) + c) : nullptr;
        rc = do_adamw_flat(P.master + a + c, P.exp_avg + a + c, P.exp_avg_sq + a + c, p16c, P.param_dtype,
                           static_cast<const char*>(ga) + c * gsz, P.grad_dtype, b - a - c, P.out + k, s);
      }
    } else {
      rc = do_adamw_flat(P.master + a, P.exp_avg + a, P.exp_avg_sq + a, p16, P.param_dtype, ga, P.grad_dtype, b - a,
                         P.out + k, s);
    }
    writer = false;
  }
  return rc;
}

}  // namespace

// ---- C ABI ---------------------------------------------------------------------

extern "C" {

int dsx_abi_version(void) { return DSX_ABI_VERSION; }

const char* dsx_last_error(void) { return g_err; }

int dsx_set_tuning(int k1_blocks_per_cu, int k2_blocks_per_cu, int k2_unroll, int nontemporal) {
  if (k1_blocks_per_cu < 1 || k1_blocks_per_cu > 32 || k2_blocks_per_cu < 0 || k2_blocks_per_cu > 64)
    return fail(DSX_EINVAL, "blocks per CU out of range");
  if (k2_unroll != 0 && k2_unroll != 2 && k2_unroll != 4 && k2_unroll != 8)
    return fail(DSX_EINVAL, "k2_unroll must be 0 (by size), 2, 4 or 8");
  g_tune.k1_blocks_per_cu = k1_blocks_per_cu;
  g_tune.k2_blocks_per_cu = k2_blocks_per_cu;
  g_tune.k2_unroll = k2_unroll;
  g_tune.nontemporal = nontemporal ? 1 : 0;
  return DSX_OK;
}

int dsx_set_tuning_k2(int k2_cu_eighths, int drain) {
  if (k2_cu_eighths < 0 || k2_cu_eighths > 8) return fail(DSX_EINVAL, "k2_cu_eighths must be in [0, 8]");
  if (drain < -1 || drain > 1) return fail(DSX_EINVAL, "drain must be -1 (by size), 0 or 1");
  g_tune.k2_cu_eighths = k2_cu_eighths;
  g_tune.k2_drain = drain;
  return DSX_OK;
}

int dsx_set_tuning_k2_chunk(int64_t chunk_elems) {
  if (chunk_elems < 0) return fail(DSX_EINVAL, "chunk_elems must be >= 0 (0: one launch)");
  if (chunk_elems > 0 && chunk_elems < (int64_t(1) << 20))
    return fail(DSX_EINVAL, "chunk_elems must be 0 or at least 2^20");
  g_tune.k2_chunk_elems = chunk_elems;
  return DSX_OK;
}

int dsx_set_tuning_fold(int64_t max_elems) {
  if (max_elems < 0) return fail(DSX_EINVAL, "max_elems must be >= 0 (0: three launches always)");
  g_tune.fold_max_elems = max_elems;
  return DSX_OK;
}

int dsx_set_tuning_multi(int k3_blocks_per_cu, int k3_unroll, int nontemporal, int drain) {
  if (k3_blocks_per_cu < 0 || k3_blocks_per_cu > 4096) return fail(DSX_EINVAL, "blocks per CU out of range");
  if (k3_unroll != 1 && k3_unroll != 2 && k3_unroll != 4) return fail(DSX_EINVAL, "k3_unroll must be 1, 2 or 4");
  if (drain < -1 || drain > 1) return fail(DSX_EINVAL, "drain must be -1 (by shape), 0 or 1");
  g_tune.k3_blocks_per_cu = k3_blocks_per_cu;
  g_tune.k3_unroll = k3_unroll;
  g_tune.k3_nontemporal = nontemporal ? 1 : 0;
  g_tune.k3_drain = drain;
  return DSX_OK;
}

int32_t dsx_suggest_partials(int64_t n) {
  const int64_t slots = n > 0 ? (n >> 3) : 0;
  const int64_t need = ceil_div(slots > 0 ? slots : 1, (int64_t)kBlock * 4);
  int64_t cap = (int64_t)cu_count() * g_tune.k1_blocks_per_cu;
  if (cap > DSX_MAX_PARTIALS) cap = DSX_MAX_PARTIALS;
  return (int32_t)(need < cap ? need : cap);
}

int64_t dsx_count_chunks(const int64_t* numels, int32_t ntensors, int64_t chunk_elems) {
  if (!numels || ntensors < 0 || chunk_elems < 8 || (chunk_elems & 7)) {
    fail(DSX_EINVAL, "dsx_count_chunks: bad arguments");
    return -1;
  }
  int64_t c = 0;
  for (int32_t i = 0; i < ntensors; ++i) {
    if (numels[i] < 0) {
      fail(DSX_EINVAL, "dsx_count_chunks: negative numel");
      return -1;
    }
    const int64_t add = ceil_div(numels[i], chunk_elems);
    if (add > INT64_MAX - c) {
      fail(DSX_EINVAL, "dsx_count_chunks: the chunk count overflows int64");
      return -1;
    }
    c += add;
  }
  return c;
}

int64_t dsx_build_chunks(const int64_t* numels, int32_t ntensors, int64_t chunk_elems, DsxChunk* out, int64_t cap) {
  const int64_t need = dsx_count_chunks(numels, ntensors, chunk_elems);
  if (need < 0) return -1;
  if (!out || cap < need) {
    fail(DSX_EINVAL, "dsx_build_chunks: capacity %lld < %lld", (long long)cap, (long long)need);
    return -1;
  }
  int64_t c = 0;
  for (int32_t i = 0; i < ntensors; ++i) {
    // By chunk index: every start is below numels[i], so nothing overflows.
    const int64_t nc = ceil_div(numels[i], chunk_elems);
    for (int64_t j = 0; j < nc; ++j) {
      const int64_t s = j * chunk_elems;
      out[c].tensor = i;
      out[c].reserved = 0;
      out[c].start = s;
      out[c].len = numels[i] - s < chunk_elems ? numels[i] - s : chunk_elems;
      ++c;
    }
  }
  return c;
}

int dsx_state_init(DsxState* state, float init_scale, int32_t hysteresis, void* stream) {
  if (!state) return fail(DSX_EINVAL, "null state");
  if (!(init_scale > 0.0f) || !__builtin_isfinite(init_scale))
    return fail(DSX_EINVAL, "initial loss scale must be finite and > 0 (got %g)", init_scale);
  if (hysteresis < 1) return fail(DSX_EINVAL, "hysteresis must be >= 1 (got %d)", hysteresis);
  hipLaunchKernelGGL(k_state_init, dim3(1), dim3(64), 0, as_stream(stream), state, init_scale, hysteresis);
  return launch_status("dsx_state_init");
}

int dsx_unscale_norm(const void* grad, int grad_dtype, int64_t n, const DsxState* state, double* partials,
                     int32_t nparts, void* stream) {
  if (!is_grad_dtype(grad_dtype))
    return fail(DSX_EINVAL, "grad dtype must be DSX_F16, DSX_BF16 or DSX_F32 (got %d)", grad_dtype);
  if (n < 0) return fail(DSX_EINVAL, "n must be >= 0");
  if (n > 0 && (!grad || !aligned16(grad))) return fail(DSX_EINVAL, "grad must be non-null and 16-byte aligned");
  if (!state) return fail(DSX_EINVAL, "null state");
  int rc = check_parts(partials, nparts);
  if (rc) return rc;
  return do_unscale_norm(grad, grad_dtype, n, state, partials, nparts, as_stream(stream));
}

int dsx_norm_partials(const void* grad, int grad_dtype, int64_t n, const DsxState* state, double norm_type,
                      double* partials, int32_t nparts, void* stream) {
  if (!is_grad_dtype(grad_dtype))
    return fail(DSX_EINVAL, "grad dtype must be DSX_F16, DSX_BF16 or DSX_F32 (got %d)", grad_dtype);
  if (n < 0) return fail(DSX_EINVAL, "n must be >= 0");
  if (n > 0 && (!grad || !aligned16(grad))) return fail(DSX_EINVAL, "grad must be non-null and 16-byte aligned");
  if (!state) return fail(DSX_EINVAL, "null state");
  int kind = 0;
  int rc = norm_kind(norm_type, &kind);
  if (!rc) rc = check_parts(partials, nparts);
  if (rc) return rc;
  return do_norm(grad_dtype, kind, false, grad, n, nullptr, nullptr, 0, state, norm_type, partials, nparts,
                 as_stream(stream));
}

int dsx_norm_partials_multi(const DsxTensorRef* tensors, const DsxChunk* chunks, int64_t nchunks, int grad_dtype,
                            const DsxState* state, double norm_type, double* partials, int32_t nparts,
                            void* stream) {
  if (!is_grad_dtype(grad_dtype))
    return fail(DSX_EINVAL, "grad dtype must be DSX_F16, DSX_BF16 or DSX_F32 (got %d)", grad_dtype);
  if (nchunks < 0 || (nchunks > 0 && (!tensors || !chunks))) return fail(DSX_EINVAL, "bad chunk table");
  if (!state) return fail(DSX_EINVAL, "null state");
  int kind = 0;
  int rc = norm_kind(norm_type, &kind);
  if (!rc) rc = check_parts(partials, nparts);
  if (rc) return rc;
  return do_norm(grad_dtype, kind, true, nullptr, 0, tensors, chunks, nchunks, state, norm_type, partials, nparts,
                 as_stream(stream));
}

int dsx_clip_prepare(const double* partials, int32_t nparts, double norm_type, double max_norm, double clip_eps,
                     DsxState* state, double* norm_out, void* stream) {
  int kind = 0;
  int rc = norm_kind(norm_type, &kind);
  if (!rc) rc = check_parts(partials, nparts);
  if (rc) return rc;
  if (!(max_norm >= 0.0)) return fail(DSX_EINVAL, "max_norm must be >= 0, got %g", max_norm);
  if (!(clip_eps >= 0.0)) return fail(DSX_EINVAL, "Invalid clip_eps: %g", clip_eps);
  if (!state || !norm_out) return fail(DSX_EINVAL, "null state or norm_out");
  hipStream_t s = as_stream(stream);
  const dim3 grid(1), blk(kBlock);
  switch (kind) {
    case kNormSq:
      hipLaunchKernelGGL(k_clip_prepare<kNormSq>, grid, blk, 0, s, partials, nparts, norm_type, max_norm, clip_eps,
                         state, norm_out);
      break;
    case kNormAbs:
      hipLaunchKernelGGL(k_clip_prepare<kNormAbs>, grid, blk, 0, s, partials, nparts, norm_type, max_norm, clip_eps,
                         state, norm_out);
      break;
    case kNormMax:
      hipLaunchKernelGGL(k_clip_prepare<kNormMax>, grid, blk, 0, s, partials, nparts, norm_type, max_norm, clip_eps,
                         state, norm_out);
      break;
    default:
      hipLaunchKernelGGL(k_clip_prepare<kNormPow>, grid, blk, 0, s, partials, nparts, norm_type, max_norm, clip_eps,
                         state, norm_out);
      break;
  }
  return launch_status("dsx_clip_prepare");
}

int dsx_finalize(const double* partials, int32_t nparts, DsxState* state, DsxScalerConfig scaler,
                 DsxAdamwHyper hyper, const double* bc_table, int32_t bc_len, DsxStepScalars* out, void* stream) {
  int rc = check_parts(partials, nparts);
  if (!rc) rc = check_scaler(scaler);
  if (!rc) rc = check_hyper(hyper);
  if (rc) return rc;
  if (!state || !out) return fail(DSX_EINVAL, "null state or scalars");
  if (bc_len < 0 || (bc_len > 0 && !bc_table)) return fail(DSX_EINVAL, "bad bias-correction table");
  return do_finalize(partials, nparts, state, scaler, one_group(hyper, bc_table, bc_len), out, as_stream(stream));
}

int dsx_finalize_groups(const double* partials, int32_t nparts, DsxState* state, DsxScalerConfig scaler,
                        const DsxAdamwHyper* hypers, const double* const* bc_tables, const int32_t* t_offsets,
                        int32_t ngroups, int32_t bc_len, DsxStepScalars* out, void* stream) {
  int rc = check_parts(partials, nparts);
  if (!rc) rc = check_scaler(scaler);
  if (rc) return rc;
  if (ngroups < 1 || ngroups > DSX_MAX_GROUPS)
    return fail(DSX_EINVAL, "ngroups must be in [1, %d] (got %d)", DSX_MAX_GROUPS, ngroups);
  if (!hypers || !bc_tables || !t_offsets) return fail(DSX_EINVAL, "null group arrays");
  if (!state || !out) return fail(DSX_EINVAL, "null state or scalars");
  if (bc_len < 0) return fail(DSX_EINVAL, "bad bias-correction table length");
  DsxGroupsDev grp = {};
  grp.ngroups = ngroups;
  grp.bc_len = bc_len;
  for (int k = 0; k < ngroups; ++k) {
    rc = check_hyper(hypers[k]);
    if (rc) return rc;
    if (bc_len > 0 && !bc_tables[k]) return fail(DSX_EINVAL, "null bias-correction table for group %d", k);
    if (t_offsets[k] < 0) return fail(DSX_EINVAL, "negative t_offset for group %d", k);
    grp.hyper[k] = hypers[k];
    grp.bc_table[k] = bc_tables[k];
    grp.t_offset[k] = t_offsets[k];
  }
  return do_finalize(partials, nparts, state, scaler, grp, out, as_stream(stream));
}

int dsx_finalize_dev(const double* partials, int32_t nparts, DsxState* state, DsxScalerConfig scaler,
                     const DsxGroupsDev* groups, int32_t max_groups, DsxStepScalars* out, void* stream) {
  int rc = check_parts(partials, nparts);
  if (!rc) rc = check_scaler(scaler);
  if (rc) return rc;
  if (!state || !out || !groups) return fail(DSX_EINVAL, "null state, scalars or groups");
  if (max_groups < 1 || max_groups > DSX_MAX_GROUPS)
    return fail(DSX_EINVAL, "max_groups must be in [1, %d] (got %d)", DSX_MAX_GROUPS, max_groups);
  hipLaunchKernelGGL(k0_finalize_dev, dim3(1), dim3(kBlock), 0, as_stream(stream), partials, nparts, state, scaler,
                     groups, max_groups, out);
  return launch_status("dsx_finalize_dev");
}

int dsx_groups_upload(const DsxGroupsDev* groups, DsxGroupsDev* dst, void* stream) {
  if (!groups || !dst) return fail(DSX_EINVAL, "null group block");
  if (reinterpret_cast<uintptr_t>(dst) & 7u) return fail(DSX_EINVAL, "dst must be 8-byte aligned");
  const DsxGroupsDev& g = *groups;
  if (g.ngroups < 1 || g.ngroups > DSX_MAX_GROUPS)
    return fail(DSX_EINVAL, "ngroups must be in [1, %d] (got %d)", DSX_MAX_GROUPS, g.ngroups);
  if (g.bc_len < 0) return fail(DSX_EINVAL, "bad bias-correction table length");
  for (int k = 0; k < g.ngroups; ++k) {
    const int rc = check_hyper(g.hyper[k]);
    if (rc) return rc;
    if (g.bc_len > 0 && !g.bc_table[k]) return fail(DSX_EINVAL, "null bias-correction table for group %d", k);
    if (g.t_offset[k] < 0) return fail(DSX_EINVAL, "negative t_offset for group %d", k);
  }
  hipLaunchKernelGGL(k_store_groups, dim3(1), dim3(64), 0, as_stream(stream), g, dst);
  return launch_status("dsx_groups_upload");
}

int dsx_adamw_flat(float* master, float* exp_avg, float* exp_avg_sq, void* param16, int param_dtype,
                   const void* grad, int grad_dtype, int64_t n, const DsxStepScalars* scalars, void* stream) {
  int rc = check_flat(master, exp_avg, exp_avg_sq, param16, param_dtype, grad, grad_dtype, n);
  if (rc) return rc;
  if (!scalars) return fail(DSX_EINVAL, "null scalars");
  return do_adamw_flat(master, exp_avg, exp_avg_sq, param16, param_dtype, grad, grad_dtype, n, scalars,
                       as_stream(stream));
}

int dsx_traffic_probe_flat(float* master, float* exp_avg, float* exp_avg_sq, void* param16, int dtype,
                           const void* grad, int64_t n, void* stream) {
  int rc = check_flat(master, exp_avg, exp_avg_sq, param16, dtype, grad, dtype, n);
  if (rc) return rc;
  if (!is16(dtype)) return fail(DSX_EINVAL, "the traffic probe takes DSX_F16 or DSX_BF16 (got %d)", dtype);
  if (!param16) return fail(DSX_EINVAL, "the traffic probe needs param16");
  if (n == 0) return DSX_OK;
  k2_dispatch(master, exp_avg, exp_avg_sq, param16, dtype, grad, dtype, n, nullptr, as_stream(stream), true);
  return launch_status("dsx_traffic_probe_flat");
}

int dsx_zero_step_flat(float* master, float* exp_avg, float* exp_avg_sq, void* param16, int param_dtype,
                       const void* grad, int grad_dtype, int64_t n, DsxState* state, DsxScalerConfig scaler,
                       DsxAdamwHyper hyper, const double* bc_table, int32_t bc_len, double* partials,
                       int32_t nparts, DsxStepScalars* out, void* stream) {
  int rc = check_zero_step(master, exp_avg, exp_avg_sq, param16, param_dtype, grad, grad_dtype, n, state, scaler,
                           hyper, bc_table, bc_len);
  if (!rc) rc = check_parts(partials, nparts);
  if (rc) return rc;
  if (!out) return fail(DSX_EINVAL, "null scalars");
  return zero_step_flat(master, exp_avg, exp_avg_sq, param16, param_dtype, grad, grad_dtype, n, state, scaler, hyper,
                        bc_table, bc_len, partials, nparts, out, as_stream(stream));
}

int dsx_zero_step_plan(const DsxFlatPlan* plan, const DsxGroupsDev* groups, void* stream) {
  if (!plan || !groups) return fail(DSX_EINVAL, "null plan or groups");
  const DsxFlatPlan& P = *plan;
  const DsxGroupsDev& G = *groups;
  int rc = check_plan(P);
  if (rc) return rc;
  if (G.ngroups != P.ngroups)
    return fail(DSX_EINVAL, "the group block holds %d groups, the plan %d", G.ngroups, P.ngroups);
  if (G.bc_len < 0) return fail(DSX_EINVAL, "bad bias-correction table length");
  for (int k = 0; k < P.ngroups; ++k) {
    rc = check_hyper(G.hyper[k]);
    if (rc) return rc;
    if (G.bc_len > 0 && !G.bc_table[k]) return fail(DSX_EINVAL, "null bias-correction table for group %d", k);
    if (G.t_offset[k] < 0) return fail(DSX_EINVAL, "negative t_offset for group %d", k);
  }
  return plan_launches(P, &G, nullptr, as_stream(stream));
}

int dsx_zero_step_dev(const DsxFlatPlan* plan, const DsxGroupsDev* groups_dev, void* stream) {
  if (!plan || !groups_dev) return fail(DSX_EINVAL, "null plan or groups");
  if (reinterpret_cast<uintptr_t>(groups_dev) & 7u) return fail(DSX_EINVAL, "groups must be 8-byte aligned");
  const int rc = check_plan(*plan);
  if (rc) return rc;
  return plan_launches(*plan, nullptr, groups_dev, as_stream(stream));
}

int dsx_zero_step_flat_noalloc(float* master, float* exp_avg, float* exp_avg_sq, void* param16, int param_dtype,
                               const void* grad, int grad_dtype, int64_t n, DsxState* state, DsxScalerConfig scaler,
                               DsxAdamwHyper hyper, const double* bc_table, int32_t bc_len, int32_t nparts,
                               DsxStepScalars* out, void* stream) {
  int rc = check_zero_step(master, exp_avg, exp_avg_sq, param16, param_dtype, grad, grad_dtype, n, state, scaler,
                           hyper, bc_table, bc_len);
  if (rc) return rc;
  if (nparts > DSX_NOALLOC_MAX_PARTIALS)
    return fail(DSX_EINVAL, "nparts %d exceeds the library scratch of %d partials", nparts, DSX_NOALLOC_MAX_PARTIALS);
  if (nparts < 0) return fail(DSX_EINVAL, "nparts must be >= 0 (0: the library's choice; got %d)", nparts);
  if (nparts == 0) {
    nparts = dsx_suggest_partials(n);
    if (nparts < 1) nparts = 1;
    if (nparts > DSX_NOALLOC_MAX_PARTIALS) nparts = DSX_NOALLOC_MAX_PARTIALS;
  }
  hipStream_t s = as_stream(stream);
  unsigned char* base = nullptr;
  rc = noalloc_scratch(s, &base);
  if (rc) return rc;
  // Every partial K0 reads is written by this step's K1 (one per block) and
  // every scalar K2 reads by this step's K0, so nothing needs clearing.
  double* partials = reinterpret_cast<double*>(base);
  DsxStepScalars* sc = out ? out : reinterpret_cast<DsxStepScalars*>(base + kScratchScalarsOffset);
  return zero_step_flat(master, exp_avg, exp_avg_sq, param16, param_dtype, grad, grad_dtype, n, state, scaler, hyper,
                        bc_table, bc_len, partials, nparts, sc, s);
}

int dsx_copy_unscale_norm(const void* src, void* dst, int grad_dtype, int64_t n, const DsxState* state,
                          double* partials, int32_t nparts, void* stream) {
  if (!is_grad_dtype(grad_dtype))
    return fail(DSX_EINVAL, "grad dtype must be DSX_F16, DSX_BF16 or DSX_F32 (got %d)", grad_dtype);
  if (n < 0) return fail(DSX_EINVAL, "n must be >= 0");
  if (n > 0 && (!src || !dst || !aligned16(src) || !aligned16(dst)))
    return fail(DSX_EINVAL, "src and dst must be non-null and 16-byte aligned");
  if (!state) return fail(DSX_EINVAL, "null state");
  int rc = check_parts(partials, nparts);
  if (rc) return rc;
  hipStream_t s = as_stream(stream);
  const dim3 grid((unsigned)nparts);
  switch (grad_dtype) {
    case DSX_BF16:
      hipLaunchKernelGGL((k1_copy_unscale_norm<DSX_BF16, 4>), grid, dim3(kBlock), 0, s, src, dst, n, state, partials);
      break;
    case DSX_F16:
      hipLaunchKernelGGL((k1_copy_unscale_norm<DSX_F16, 4>), grid, dim3(kBlock), 0, s, src, dst, n, state, partials);
      break;
    default:
      hipLaunchKernelGGL((k1_copy_unscale_norm<DSX_F32, 4>), grid, dim3(kBlock), 0, s, src, dst, n, state, partials);
      break;
  }
  return launch_status("dsx_copy_unscale_norm");
}

int dsx_reduce_segments(const double* partials, const int64_t* offsets, int32_t nseg, double* out, void* stream) {
  if (nseg < 1 || nseg > DSX_MAX_PARTIALS)
    return fail(DSX_EINVAL, "nseg must be in [1, %d] (got %d)", DSX_MAX_PARTIALS, nseg);
  if (!partials || !offsets || !out) return fail(DSX_EINVAL, "null partials, offsets or out");
  hipLaunchKernelGGL(k_reduce_segments, dim3((unsigned)nseg), dim3(kBlock), 0, as_stream(stream), partials, offsets,
                     out);
  return launch_status("dsx_reduce_segments");
}

int dsx_unscale_norm_multi(const DsxTensorRef* tensors, const DsxChunk* chunks, int64_t nchunks, int grad_dtype,
                           const DsxState* state, double* partials, int32_t nparts, void* stream) {
  if (!is_grad_dtype(grad_dtype))
    return fail(DSX_EINVAL, "grad dtype must be DSX_F16, DSX_BF16 or DSX_F32 (got %d)", grad_dtype);
  if (nchunks < 0 || (nchunks > 0 && (!tensors || !chunks))) return fail(DSX_EINVAL, "bad chunk table");
  if (!state) return fail(DSX_EINVAL, "null state");
  int rc = check_parts(partials, nparts);
  if (rc) return rc;
  return do_unscale_norm_multi(tensors, chunks, nchunks, grad_dtype, state, partials, nparts, as_stream(stream),
                               nullptr);
}

int dsx_adamw_multi(const DsxTensorRef* tensors, const DsxChunk* chunks, int64_t nchunks, int param_dtype,
                    int grad_dtype, const DsxStepScalars* scalars, void* stream) {
  if (!is_grad_dtype(grad_dtype))
    return fail(DSX_EINVAL, "grad dtype must be DSX_F16, DSX_BF16 or DSX_F32 (got %d)", grad_dtype);
  if (!is16(param_dtype)) return fail(DSX_EINVAL, "param16 dtype must be DSX_F16 or DSX_BF16 (got %d)", param_dtype);
  if (nchunks < 0 || (nchunks > 0 && (!tensors || !chunks))) return fail(DSX_EINVAL, "bad chunk table");
  if (!scalars) return fail(DSX_EINVAL, "null scalars");
  return do_adamw_multi(tensors, chunks, nchunks, param_dtype, grad_dtype, scalars, as_stream(stream));
}

int dsx_zero_step_multi(const DsxTensorRef* tensors, const DsxChunk* chunks, int64_t nchunks, int64_t numel,
                        int param_dtype, int grad_dtype, DsxState* state, DsxScalerConfig scaler,
                        const DsxGroupsDev* groups, double* partials, int32_t nparts, DsxStepScalars* out,
                        void* stream) {
  if (!is_grad_dtype(grad_dtype))
    return fail(DSX_EINVAL, "grad dtype must be DSX_F16, DSX_BF16 or DSX_F32 (got %d)", grad_dtype);
  if (!is16(param_dtype)) return fail(DSX_EINVAL, "param16 dtype must be DSX_F16 or DSX_BF16 (got %d)", param_dtype);
  if (nchunks < 0 || (nchunks > 0 && (!tensors || !chunks))) return fail(DSX_EINVAL, "bad chunk table");
  if (numel < 0) return fail(DSX_EINVAL, "numel must be >= 0");
  if (!state || !out || !groups) return fail(DSX_EINVAL, "null state, scalars or groups");
  int rc = check_parts(partials, nparts);
  if (!rc) rc = check_scaler(scaler);
  if (rc) return rc;
  const DsxGroupsDev& G = *groups;
  if (G.ngroups < 1 || G.ngroups > DSX_MAX_GROUPS)
    return fail(DSX_EINVAL, "ngroups must be in [1, %d] (got %d)", DSX_MAX_GROUPS, G.ngroups);
  if (G.bc_len < 0) return fail(DSX_EINVAL, "bad bias-correction table length");
  for (int k = 0; k < G.ngroups; ++k) {
    rc = check_hyper(G.hyper[k]);
    if (rc) return rc;
    if (G.bc_len > 0 && !G.bc_table[k]) return fail(DSX_EINVAL, "null bias-correction table for group %d", k);
    if (G.t_offset[k] < 0) return fail(DSX_EINVAL, "negative t_offset for group %d", k);
  }
  hipStream_t s = as_stream(stream);
  // Two launches where the fold applies and the list takes K3's one-chunk-
  // per-block shape; else K1, K0, K3.
  const bool fold = nchunks > 0 && fold_applies(numel, nparts) && nchunks <= kK3OneChunkPerCu * cu_count();
  rc = do_unscale_norm_multi(tensors, chunks, nchunks, grad_dtype, state, partials, nparts, s,
                             fold ? state : nullptr);
  if (rc) return rc;
  if (!fold) {
    rc = do_finalize(partials, nparts, state, scaler, G, out, s);
    if (!rc) rc = do_adamw_multi(tensors, chunks, nchunks, param_dtype, grad_dtype, out, s);
    return rc;
  }
  const dim3 grid((unsigned)(nchunks + 1));  // one chunk per block, and the writer
  switch (grad_dtype) {
    case DSX_BF16: launch_k3_fold<DSX_BF16>(param_dtype, grid, tensors, chunks, nchunks, partials, nparts, state,
                                            scaler, G, out, s); break;
    case DSX_F16: launch_k3_fold<DSX_F16>(param_dtype, grid, tensors, chunks, nchunks, partials, nparts, state,
                                          scaler, G, out, s); break;
    default: launch_k3_fold<DSX_F32>(param_dtype, grid, tensors, chunks, nchunks, partials, nparts, state, scaler,
                                     G, out, s); break;
  }
  return launch_status("dsx_zero_step_multi (finalize folded in)");
}

}  // extern "C"
