/*
 * A plain C caller of libdsx.so: no Python, no torch in the process. It is
 * what a C or C++ host (a custom ZeRO stage that owns its flat fp32 buffers,
 * Src/zero/stage2.py:108-193) would write against include/dsx.h: device
 * buffers from hipMalloc, the state from dsx_state_init, the bias-correction
 * table computed on the host in double as torch computes it
 * (torch/optim/adam.py: 1 - beta1**t and (1 - beta2**t)**0.5), then one
 * dsx_zero_step_flat call per step on a stream of its own -- and, on a
 * second copy of the buffers, dsx_zero_step_flat_noalloc.
 *
 * usage: dsx_c_caller <n> <dtype 1 (fp16, dynamic loss scale) | 2 (bf16)>
 *                     <steps> <outdir> [fold_max_elems]
 * fold_max_elems, when given, goes to dsx_set_tuning_fold first: 0 makes
 * every one-call step run K1, K0 and K2 as three launches.
 * Writes to outdir: master0.f32 (the initial master), grads.u16 (the 16-bit
 * grads of every step, step after step), master.f32, exp_avg.f32,
 * exp_avg_sq.f32, param16.u16 (after the last step) and states.bin (the
 * 64-byte DsxState after every step). Step 1's grads hold an inf. Prints
 * "noalloc identical" when the no-allocation copy ended bit-identical.
 * Exit status 0 on success.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "dsx.h"

#define CHECK_HIP(x)                                                              \
  do {                                                                            \
    hipError_t e_ = (x);                                                          \
    if (e_ != hipSuccess) {                                                       \
      fprintf(stderr, "%s:%d: %s\n", __FILE__, __LINE__, hipGetErrorString(e_));  \
      exit(2);                                                                    \
    }                                                                             \
  } while (0)

#define CHECK_DSX(x)                                                              \
  do {                                                                            \
    int r_ = (x);                                                                 \
    if (r_ != DSX_OK) {                                                           \
      fprintf(stderr, "%s:%d: status %d: %s\n", __FILE__, __LINE__, r_,           \
              dsx_last_error());                                                  \
      exit(3);                                                                    \
    }                                                                             \
  } while (0)

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;

/* xorshift64*, then a sum of four uniforms: roughly N(0, 1/3), enough for
 * synthetic weights and grads */
static double next_u01(void) {
  rng_state ^= rng_state >> 12;
  rng_state ^= rng_state << 25;
  rng_state ^= rng_state >> 27;
  return (double)((rng_state * 0x2545F4914F6CDD1Dull) >> 11) * (1.0 / 9007199254740992.0);
}

static float next_normalish(void) {
  return (float)(next_u01() + next_u01() + next_u01() + next_u01() - 2.0);
}

/* fp32 -> fp16 / bf16, round to nearest even (finite inputs well inside range) */
static uint16_t to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

static uint16_t to_f16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  const uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
  if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds past 65504 */
  if (a >= 0x38800000u)                                   /* normal: rebias the exponent, round at bit 13 */
    return (uint16_t)(sign | ((a - 0x38000000u + 0xFFFu + ((a >> 13) & 1u)) >> 13));
  return (uint16_t)(sign | (uint32_t)nearbyintf(fabsf(x) * 16777216.0f)); /* subnormal: units of 2^-24 */
}

static void write_file(const char* dir, const char* name, const void* p, size_t bytes, const char* mode) {
  char path[4096];
  snprintf(path, sizeof path, "%s/%s", dir, name);
  FILE* f = fopen(path, mode);
  if (!f || fwrite(p, 1, bytes, f) != bytes) {
    fprintf(stderr, "cannot write %s\n", path);
    exit(4);
  }
  fclose(f);
}

typedef struct {
  float *p, *m, *v;
  uint16_t *p16, *g;
  DsxState* st;
  DsxStepScalars* out;
} Side;

static void side_init(Side* s, int64_t n, const float* master0, const uint16_t* p16_0, float scale, int hyst,
                      hipStream_t stream) {
  CHECK_HIP(hipMalloc((void**)&s->p, 4 * n));
  CHECK_HIP(hipMalloc((void**)&s->m, 4 * n));
  CHECK_HIP(hipMalloc((void**)&s->v, 4 * n));
  CHECK_HIP(hipMalloc((void**)&s->p16, 2 * n));
  CHECK_HIP(hipMalloc((void**)&s->g, 2 * n));
  CHECK_HIP(hipMalloc((void**)&s->st, sizeof(DsxState)));
  CHECK_HIP(hipMalloc((void**)&s->out, sizeof(DsxStepScalars)));
  CHECK_HIP(hipMemcpy(s->p, master0, 4 * n, hipMemcpyHostToDevice));
  CHECK_HIP(hipMemset(s->m, 0, 4 * n));
  CHECK_HIP(hipMemset(s->v, 0, 4 * n));
  CHECK_HIP(hipMemcpy(s->p16, p16_0, 2 * n, hipMemcpyHostToDevice));
  CHECK_DSX(dsx_state_init(s->st, scale, hyst, stream));
}

static int same(const void* a, const void* b, size_t bytes, void* ha, void* hb) {
  CHECK_HIP(hipMemcpy(ha, a, bytes, hipMemcpyDeviceToHost));
  CHECK_HIP(hipMemcpy(hb, b, bytes, hipMemcpyDeviceToHost));
  return memcmp(ha, hb, bytes) == 0;
}

int main(int argc, char** argv) {
  if (argc != 5 && argc != 6) {
    fprintf(stderr, "usage: %s n dtype steps outdir [fold_max_elems]\n", argv[0]);
    return 1;
  }
  const int64_t n = atoll(argv[1]);
  const int dt = atoi(argv[2]);
  const int steps = atoi(argv[3]);
  const char* dir = argv[4];
  if (n < 1 || (dt != DSX_F16 && dt != DSX_BF16) || steps < 2) {
    fprintf(stderr, "bad arguments\n");
    return 1;
  }
  if (dsx_abi_version() != DSX_ABI_VERSION) {
    fprintf(stderr, "ABI %d, header %d\n", dsx_abi_version(), DSX_ABI_VERSION);
    return 1;
  }
  if (argc == 6) CHECK_DSX(dsx_set_tuning_fold((int64_t)atoll(argv[5])));
  CHECK_HIP(hipSetDevice(0));
  hipStream_t stream;
  CHECK_HIP(hipStreamCreate(&stream));

  const int fp16 = dt == DSX_F16;
  DsxScalerConfig scaler;
  memset(&scaler, 0, sizeof scaler);
  scaler.mode = fp16 ? DSX_SCALE_DYNAMIC : DSX_SCALE_NONE;
  scaler.window = 2;
  scaler.hysteresis = 1;
  scaler.min_scale = 1.0f;
  scaler.growth_factor = 2.0f;
  scaler.backoff_factor = 0.5f;
  const float scale0 = fp16 ? 4096.0f : 1.0f;
  DsxAdamwHyper hyper = {1e-3, 0.9, 0.95, 1e-8, 0.1, 1.0, 1e-6};

  /* bias-correction table, as torch evaluates it on the host */
  const int bc_len = 1024;
  double* bc_host = (double*)malloc(sizeof(double) * 2 * bc_len);
  for (int t = 1; t <= bc_len; ++t) {
    bc_host[2 * (t - 1)] = 1.0 - pow(hyper.beta1, (double)t);
    bc_host[2 * (t - 1) + 1] = pow(1.0 - pow(hyper.beta2, (double)t), 0.5);
  }
  double* bc;
  CHECK_HIP(hipMalloc((void**)&bc, sizeof(double) * 2 * bc_len));
  CHECK_HIP(hipMemcpy(bc, bc_host, sizeof(double) * 2 * bc_len, hipMemcpyHostToDevice));

  float* master0 = (float*)malloc(4 * n);
  uint16_t* p16_0 = (uint16_t*)malloc(2 * n);
  for (int64_t i = 0; i < n; ++i) {
    master0[i] = 0.03f * next_normalish();
    p16_0[i] = fp16 ? to_f16(master0[i]) : to_bf16(master0[i]);
  }
  write_file(dir, "master0.f32", master0, 4 * n, "wb");

  Side a, b; /* a: dsx_zero_step_flat with caller scratch; b: the no-allocation variant */
  side_init(&a, n, master0, p16_0, scale0, 1, stream);
  side_init(&b, n, master0, p16_0, scale0, 1, stream);
  const int32_t nparts = dsx_suggest_partials(n);
  double* partials;
  CHECK_HIP(hipMalloc((void**)&partials, sizeof(double) * nparts));

  uint16_t* g16 = (uint16_t*)malloc(2 * n);
  DsxState st;
  char gname[] = "grads.u16";
  char sname[] = "states.bin";
  for (int k = 0; k < steps; ++k) {
    CHECK_HIP(hipMemcpy(&st, a.st, sizeof st, hipMemcpyDeviceToHost));
    for (int64_t i = 0; i < n; ++i) {
      const float g = 2e-3f * next_normalish() * st.scale;
      g16[i] = fp16 ? to_f16(g) : to_bf16(g);
    }
    if (k == 1) g16[n / 2] = fp16 ? 0x7C00u : 0x7F80u; /* +inf: the step is skipped */
    write_file(dir, gname, g16, 2 * n, k ? "ab" : "wb");
    CHECK_HIP(hipMemcpy(a.g, g16, 2 * n, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(b.g, g16, 2 * n, hipMemcpyHostToDevice));
    CHECK_DSX(dsx_zero_step_flat(a.p, a.m, a.v, a.p16, dt, a.g, dt, n, a.st, scaler, hyper, bc, bc_len, partials,
                                 nparts, a.out, stream));
    CHECK_DSX(dsx_zero_step_flat_noalloc(b.p, b.m, b.v, b.p16, dt, b.g, dt, n, b.st, scaler, hyper, bc, bc_len,
                                         nparts, b.out, stream));
    CHECK_HIP(hipStreamSynchronize(stream));
    CHECK_HIP(hipMemcpy(&st, a.st, sizeof st, hipMemcpyDeviceToHost));
    write_file(dir, sname, &st, sizeof st, k ? "ab" : "wb");
  }

  float* h = (float*)malloc(4 * n);
  float* h2 = (float*)malloc(4 * n);
  CHECK_HIP(hipMemcpy(h, a.p, 4 * n, hipMemcpyDeviceToHost));
  write_file(dir, "master.f32", h, 4 * n, "wb");
  CHECK_HIP(hipMemcpy(h, a.m, 4 * n, hipMemcpyDeviceToHost));
  write_file(dir, "exp_avg.f32", h, 4 * n, "wb");
  CHECK_HIP(hipMemcpy(h, a.v, 4 * n, hipMemcpyDeviceToHost));
  write_file(dir, "exp_avg_sq.f32", h, 4 * n, "wb");
  CHECK_HIP(hipMemcpy(h, a.p16, 2 * n, hipMemcpyDeviceToHost));
  write_file(dir, "param16.u16", h, 2 * n, "wb");

  const int ident = same(a.p, b.p, 4 * n, h, h2) && same(a.m, b.m, 4 * n, h, h2) && same(a.v, b.v, 4 * n, h, h2) &&
                    same(a.p16, b.p16, 2 * n, h, h2) && same(a.st, b.st, sizeof(DsxState), h, h2) &&
                    same(a.out, b.out, sizeof(DsxStepScalars), h, h2);
  printf(ident ? "noalloc identical\n" : "noalloc differs\n");
  return ident ? 0 : 5;
}
