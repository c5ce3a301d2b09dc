/*
 * dsx_oracle.c -- CPU restatement of the ZeRO optimizer step, used ONLY as a
 * checker (tests/, __graft_entry__.smoke(), bench.py's cpu_baseline leg).
 * Nothing in the product links or calls this file.
 *
 * What it restates, and where the reference defines it:
 *   - squared L2 norm of the unscaled grads, summed in fp64:
 *       Src/zero/utils.py:126-154 (compute_norm), Src/zero/stage2.py:683-707
 *   - unscale by the inverse loss scale and non-finite detection:
 *       Src/zero/optimizer.py:236-242, 276-298 (GradScaler.unscale_ semantics,
 *       torch/amp/grad_scaler.py:235-286)
 *   - clipping g *= max_norm / (norm + 1e-6) iff norm > max_norm:
 *       Src/zero/utils.py:187-216
 *   - AdamW (decoupled weight decay) with the per-op rounding of
 *       torch.optim.AdamW on a GPU, called by the reference at
 *       Src/zero/stage1.py:522-525, Src/zero/stage2.py:609-612; on GPU
 *       tensors torch defaults to the multi-tensor path (adam.py:938),
 *       torch/optim/adam.py:554-800 (_multi_tensor_adam):
 *         p *= f32(1 - lr*wd)                         adam.py:692
 *         m  = lerp(m, g, f32(1 - beta1))             adam.py:705-707
 *              (one fused multiply-add: fma(w, g - m, m), or for
 *               |w| >= 0.5 g - (g - m) * (1 - w) as fma(-(g - m), 1 - w, g),
 *               torch/include/ATen/native/Lerp.h:21-35)
 *         v  = fma(f32(1 - beta2), g * g, v * beta2)  adam.py:709, 722-724
 *         d  = sqrt(v) / f32(bc2_sqrt) + f32(eps)     adam.py:781, 791-794
 *         p  = fma(f32(-lr/bc1), m / d, p)            adam.py:779, 795-800
 *   - the 16-bit cast of the updated fp32 master (round to nearest even).
 *
 * Built with -ffp-contract=off so that every operation rounds on its own;
 * fmaf() is called exactly where torch's GPU kernels fuse (measured bit for
 * bit against torch on MI355X; tests/golden/adamw_torch_gpu.npz). sqrtf()
 * and '/' are IEEE correctly rounded, as torch's GPU sqrt and division are.
 * torch's CPU kernels round differently (addcmul as fma((1-b2)*g, g, v*b2),
 * addcdiv as p + (s*m)/d, MKL's sqrt), so against torch on a CPU the oracle
 * agrees within a few ulp rather than bit for bit.
 *
 * The fp16/bf16 conversions are written from the IEEE 754 binary16 and
 * bfloat16 definitions, without hardware conversion instructions.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define DSXO_F32 0
#define DSXO_F16 1
#define DSXO_BF16 2

typedef struct DsxoScalars {
  float inv_scale, clip_coef, decay, w1, w1c, b2, val2, eps, bc2s, nss;
} DsxoScalars;

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* binary16 -> binary32, exact. */
float dsxo_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  const uint32_t man = h & 0x3FFu;
  if (exp == 0x1Fu) return u2f(sign | 0x7F800000u | (man << 13)); /* inf / NaN */
  if (exp != 0) return u2f(sign | ((exp + 112u) << 23) | (man << 13));
  /* zero or subnormal: man * 2^-24 is exact in binary32 */
  const float mag = (float)man * 0x1p-24f;
  return sign ? -mag : mag;
}

float dsxo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* binary32 -> binary16, round to nearest, ties to even. NaN -> sign|0x7E00. */
uint16_t dsxo_f32_to_f16(float x) {
  const uint32_t u = f2u(x);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
  if (a == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
  const int e = (int)(a >> 23) - 127; /* unbiased exponent */
  if (e > 15) return (uint16_t)(sign | 0x7C00u);
  if (e >= -14) {
    /* normal range of binary16: keep 10 of 23 mantissa bits */
    uint32_t mant = (a & 0x7FFFFFu) | 0x800000u; /* 24 bits */
    uint32_t q = mant >> 13, rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1;
    uint32_t exp16 = (uint32_t)(e + 15);
    if (q == 0x800u) { q = 0x400u; exp16 += 1; } /* mantissa carried out */
    if (exp16 >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | (exp16 << 10) | (q & 0x3FFu));
  }
  if (e < -25) return (uint16_t)sign; /* below half the smallest subnormal */
  /* subnormal binary16: value = q * 2^-24 */
  const uint32_t mant = (a & 0x7FFFFFu) | 0x800000u; /* value = mant * 2^(e-23) */
  const int shift = -e - 1;                          /* 2^(e-23) / 2^-24 = 2^(e+1) */
  uint32_t q = mant >> shift;
  const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1;
  return (uint16_t)(sign | q); /* q == 0x400 rolls into the smallest normal */
}

/* binary32 -> bfloat16, round to nearest, ties to even. NaN -> 0x7FC0. */
uint16_t dsxo_f32_to_bf16(float x) {
  const uint32_t u = f2u(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  const uint32_t hi = u >> 16, lo = u & 0xFFFFu;
  uint32_t r = hi;
  if (lo > 0x8000u || (lo == 0x8000u && (hi & 1u))) r += 1; /* may carry into inf: correct */
  return (uint16_t)r;
}

/* Grad element i as fp32: 16-bit storage widened exactly, or fp32 as is. */
static inline float load_grad(const void* g, int64_t i, int dt) {
  if (dt == DSXO_F32) return ((const float*)g)[i];
  const uint16_t h = ((const uint16_t*)g)[i];
  return dt == DSXO_BF16 ? dsxo_bf16_to_f32(h) : dsxo_f16_to_f32(h);
}
/* Sum over i of (double)(f32(g[i]) * inv_scale)^2 in index order, with
 * Neumaier's compensated summation so that the result is accurate to a few
 * ulp of fp64 even over 10^9 terms (a plain running sum drifts ~1e-10
 * relative there). Each square is exact in fp64. Non-finite iff some unscaled
 * grad is inf or NaN. */
double dsxo_sumsq(const void* g, int dt, int64_t n, float inv_scale) {
  double s = 0.0, c = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    const float a = load_grad(g, i, dt) * inv_scale;
    const double x = (double)a * (double)a;
    const double t = s + x;
    if (!isfinite(t)) { s = t; c = 0.0; continue; }
    if (fabs(s) >= fabs(x)) c += (s - t) + x;
    else c += (x - t) + s;
    s = t;
  }
  return isfinite(s) ? s + c : s;
}

/* Same sum, split into `nblocks` contiguous blocks summed separately and then
 * added in block order -- a second summation order for cross-checks. */
double dsxo_sumsq_blocked(const void* g, int dt, int64_t n, float inv_scale, int64_t nblocks) {
  double total = 0.0;
  if (nblocks < 1) nblocks = 1;
  const int64_t per = (n + nblocks - 1) / nblocks;
  for (int64_t b = 0; b < nblocks; ++b) {
    const int64_t lo = b * per, hi = lo + per < n ? lo + per : n;
    if (lo >= n) break;
    const char* base = (const char*)g + lo * (dt == DSXO_F32 ? 4 : 2);
    total += dsxo_sumsq(base, dt, hi - lo, inv_scale);
  }
  return total;
}

/* dsxo_sumsq_blocked with the blocks summed in parallel (OpenMP) and then
 * added in block order: the same value, bit for bit, on any thread count.
 * Used where the oracle is timed (the CPU baseline). */
double dsxo_sumsq_parallel(const void* g, int dt, int64_t n, float inv_scale, int64_t nblocks) {
  enum { kMaxBlocks = 4096 };
  double part[kMaxBlocks];
  if (nblocks < 1) nblocks = 1;
  if (nblocks > kMaxBlocks) nblocks = kMaxBlocks;
  const int64_t per = (n + nblocks - 1) / nblocks;
  const size_t esz = dt == DSXO_F32 ? 4 : 2;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t b = 0; b < nblocks; ++b) {
    const int64_t lo = b * per, hi = lo + per < n ? lo + per : n;
    part[b] = lo < n ? dsxo_sumsq((const char*)g + (size_t)lo * esz, dt, hi - lo, inv_scale) : 0.0;
  }
  double total = 0.0;
  for (int64_t b = 0; b < nblocks; ++b) {
    if (b * per >= n) break;
    total += part[b];
  }
  return total;
}

/* One element of the step. `small` selects lerp's form (|w1| < 0.5); it is
 * a constant at each call site, so the branch leaves the loops below. */
static inline void step_elt(float graw, float* p, float* m, float* v, const DsxoScalars* s, int small) {
  float g = graw * s->inv_scale;
  g = g * s->clip_coef;
  float pp = *p * s->decay;
  const float d = g - *m;
  const float mm = small ? fmaf(s->w1, d, *m) : fmaf(-d, s->w1c, g);
  float vv = *v * s->b2;
  vv = fmaf(s->val2, g * g, vv);
  const float den = sqrtf(vv) / s->bc2s + s->eps;
  pp = fmaf(s->nss, mm / den, pp);
  *p = pp;
  *m = mm;
  *v = vv;
}

enum { kChunk = 512 };

/* Elements [0, len) of one chunk: grads widened into a local array, the
 * element math in a loop without branches (vectorised by the compiler; the
 * arithmetic and its rounding are those of step_elt), then the cast. */
static void adamw_chunk(float* restrict p, float* restrict m, float* restrict v, uint16_t* restrict p16, int pdt,
                        const void* g, int gdt, int64_t len, const DsxoScalars* s, int small) {
  float gw[kChunk];
  if (gdt == DSXO_BF16) {
    const uint16_t* h = (const uint16_t*)g;
    for (int64_t i = 0; i < len; ++i) gw[i] = u2f((uint32_t)h[i] << 16);
  } else {
    for (int64_t i = 0; i < len; ++i) gw[i] = load_grad(g, i, gdt);
  }
  if (small) {
    for (int64_t i = 0; i < len; ++i) step_elt(gw[i], p + i, m + i, v + i, s, 1);
  } else {
    for (int64_t i = 0; i < len; ++i) step_elt(gw[i], p + i, m + i, v + i, s, 0);
  }
  if (!p16) return;
  if (pdt == DSXO_BF16) {
    for (int64_t i = 0; i < len; ++i) p16[i] = dsxo_f32_to_bf16(p[i]);
  } else {
    for (int64_t i = 0; i < len; ++i) p16[i] = dsxo_f32_to_f16(p[i]);
  }
}

/* One AdamW step over n elements, in place; p16 (may be NULL) receives the
 * cast master. Grads are 16-bit storage (gdt F16/BF16) or fp32 (gdt F32).
 * Elements are independent, so chunks run in parallel. */
void dsxo_adamw(float* p, float* m, float* v, uint16_t* p16, int pdt, const void* g, int gdt, int64_t n,
                const DsxoScalars* s) {
  const int small = fabsf(s->w1) < 0.5f;
  const size_t gsz = gdt == DSXO_F32 ? 4 : 2;
  const int64_t nchunks = (n + kChunk - 1) / kChunk;
#pragma omp parallel for schedule(static)
  for (int64_t c = 0; c < nchunks; ++c) {
    const int64_t lo = c * kChunk, len = n - lo < kChunk ? n - lo : kChunk;
    adamw_chunk(p + lo, m + lo, v + lo, p16 ? p16 + lo : NULL, pdt, (const char*)g + (size_t)lo * gsz, gdt, len, s,
                small);
  }
}

/* Array conversions used by the tests. */
void dsxo_cast_f32(const float* x, uint16_t* out, int dt, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = dt == DSXO_BF16 ? dsxo_f32_to_bf16(x[i]) : dsxo_f32_to_f16(x[i]);
}

void dsxo_widen(const uint16_t* h, float* out, int dt, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = load_grad(h, i, dt);
}

int dsxo_num_threads(void) {
#ifdef _OPENMP
  extern int omp_get_max_threads(void);
  return omp_get_max_threads();
#else
  return 1;
#endif
}
