/*
 * mxq_oracle.c — CPU oracle for the MLX affine group-quantized linear.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product path). See
 * mxq_oracle.h for what each function restates and how it is pinned.
 * Build: oracle/Makefile (gcc -O3 -fopenmp, x86-64-v3).
 */
#include "mxq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int orc_version(void) { return 1; }

/* ------------------------------------------------------------------------ */
/* generator                                                                 */
/* ------------------------------------------------------------------------ */

#define SM_GAMMA 0x9E3779B97F4A7C15ULL

static inline uint64_t sm_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

uint64_t orc_splitmix64_next(uint64_t* state) {
  *state += SM_GAMMA;
  return sm_mix(*state);
}

/* The i-th output of a splitmix64 stream seeded with `seed` is
 * mix(seed + (i+1)*gamma), so pairs can be generated independently. */
static inline void bm_pair(uint64_t seed, int64_t pair, double* z0, double* z1) {
  uint64_t a = sm_mix(seed + (uint64_t)(2 * pair + 1) * SM_GAMMA);
  uint64_t b = sm_mix(seed + (uint64_t)(2 * pair + 2) * SM_GAMMA);
  double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0,1] */
  double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);         /* [0,1) */
  double r = sqrt(-2.0 * log(u1));
  double t = 6.283185307179586 * u2;
  *z0 = r * cos(t);
  *z1 = r * sin(t);
}

void orc_normal_f32(uint64_t seed, int64_t n, double mean, double std, float* out) {
  int64_t np = (n + 1) / 2;
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < np; ++p) {
    double z0, z1;
    bm_pair(seed, p, &z0, &z1);
    out[2 * p] = (float)(mean + std * z0);
    if (2 * p + 1 < n) out[2 * p + 1] = (float)(mean + std * z1);
  }
}

void orc_normal_bf16(uint64_t seed, int64_t n, double mean, double std, uint16_t* out) {
  int64_t np = (n + 1) / 2;
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < np; ++p) {
    double z0, z1;
    bm_pair(seed, p, &z0, &z1);
    out[2 * p] = orc_bf16_rne((float)(mean + std * z0));
    if (2 * p + 1 < n) out[2 * p + 1] = orc_bf16_rne((float)(mean + std * z1));
  }
}

/* ------------------------------------------------------------------------ */
/* bf16                                                                      */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t orc_bf16_rne(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) /* NaN */
    return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

void orc_bf16_to_f32_n(const uint16_t* in, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(in[i]);
}

void orc_f32_to_bf16_n(const float* in, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_bf16_rne(in[i]);
}

/* ------------------------------------------------------------------------ */
/* layout                                                                    */
/* ------------------------------------------------------------------------ */

static int bits_ok(int bits) {
  return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8;
}

static int layout_ok(int64_t N, int64_t K, int bits) {
  return bits_ok(bits) && N >= 0 && K >= 0 && (K * bits) % 32 == 0;
}

/* Definition (bit by bit): stream bit p = k*bits + j of row n holds bit j of
 * q[n,k]; stream bit p lives in word p/32 at bit p%32. */
int orc_pack_bitwise(const uint8_t* codes, int64_t N, int64_t K, int bits, uint32_t* wq) {
  if (!layout_ok(N, K, bits)) return -1;
  int64_t W = K * bits / 32;
  memset(wq, 0, (size_t)(N * W) * sizeof(uint32_t));
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      unsigned c = codes[n * K + k];
      for (int j = 0; j < bits; ++j) {
        int64_t p = k * bits + j;
        if ((c >> j) & 1u) wq[n * W + p / 32] |= 1u << (p % 32);
      }
    }
  return 0;
}

/* Word-wise: append codes LSB-first to a 64-bit accumulator, emit 32 bits at a
 * time. Must agree with orc_pack_bitwise bit-exactly. */
int orc_pack_words(const uint8_t* codes, int64_t N, int64_t K, int bits, uint32_t* wq) {
  if (!layout_ok(N, K, bits)) return -1;
  int64_t W = K * bits / 32;
  uint32_t mask = (1u << bits) - 1u;
  for (int64_t n = 0; n < N; ++n) {
    uint64_t acc = 0;
    int nacc = 0;
    int64_t w = 0;
    for (int64_t k = 0; k < K; ++k) {
      acc |= (uint64_t)(codes[n * K + k] & mask) << nacc;
      nacc += bits;
      if (nacc >= 32) {
        wq[n * W + w++] = (uint32_t)acc;
        acc >>= 32;
        nacc -= 32;
      }
    }
  }
  return 0;
}

static inline unsigned code_at(const uint32_t* row, int64_t k, int bits) {
  int64_t p = k * bits;
  int64_t w = p >> 5;
  int off = (int)(p & 31);
  uint64_t v = row[w];
  if (off + bits > 32) v |= (uint64_t)row[w + 1] << 32;
  return (unsigned)((v >> off) & ((1u << bits) - 1u));
}

int orc_unpack(const uint32_t* wq, int64_t N, int64_t K, int bits, uint8_t* codes) {
  if (!layout_ok(N, K, bits)) return -1;
  int64_t W = K * bits / 32;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) codes[n * K + k] = (uint8_t)code_at(wq + n * W, k, bits);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* tiled layout                                                              */
/* ------------------------------------------------------------------------ */

int64_t orc_tiled_bytes(int64_t N, int64_t K, int gs, int bits) {
  if (N < 0 || K < 0 || K % 64 != 0 || (gs != 32 && gs != 64 && gs != 128)) return -1;
  if (bits != 2 && bits != 3 && bits != 4 && bits != 5 && bits != 6 && bits != 8) return -1;
  int64_t rec = 512 * (int64_t)bits + 256 * (gs == 32 ? 2 : 1);
  return (N + 63) / 64 * (K / 64) * rec;
}

/* byte offset, inside a record, of word j of unit u in half h */
static int64_t tiled_word_offset(int bits, int h, int u, int j) {
  int64_t half = (int64_t)h * 256 * bits;
  int full = bits / 4, rem = bits % 4;
  if (j < 4 * full) return half + (j / 4) * 1024 + u * 16 + (j % 4) * 4;
  return half + full * 1024 + u * 4 * rem + (j - 4 * full) * 4;
}

int orc_tile(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases, int64_t N,
             int64_t K, int gs, int bits, uint8_t* out) {
  int64_t total = orc_tiled_bytes(N, K, gs, bits);
  if (total < 0) return -1;
  memset(out, 0, (size_t)total);
  const int64_t W = K * bits / 32, G = K / gs;
  const int64_t rec = 512 * (int64_t)bits + 256 * (gs == 32 ? 2 : 1);
  const int gps = gs == 32 ? 2 : 1;
  for (int64_t n = 0; n < N; ++n) {
    const int64_t rb = n / 64;
    const int h = (int)((n % 64) / 32), r = (int)(n % 32);
    for (int64_t k = 0; k < K; ++k) {
      const int64_t kk = k / 64;
      const int g = (int)((k % 64) / 32);
      const int u = r + 32 * g;
      uint8_t* R = out + (kk * ((N + 63) / 64) + rb) * rec; /* step-major records */
      uint32_t q = code_at(wq + n * W, k, bits);
      for (int t = 0; t < bits; ++t) {
        int pos = (int)(k % 32) * bits + t; /* bit position in the unit's run */
        uint32_t* word = (uint32_t*)(R + tiled_word_offset(bits, h, u, pos / 32));
        *word |= ((q >> t) & 1u) << (pos % 32);
      }
      if (k % gs == 0 || k % 32 == 0) {
        /* the dword for (row, code half) names the group holding its codes */
        int entry = (h * 32 + r) * gps + (gps == 2 ? g : 0);
        if (gps == 2 || g == 0) {
          uint32_t* e = (uint32_t*)(R + 512 * (int64_t)bits) + entry;
          int64_t grp = k / gs;
          *e = (uint32_t)scales[n * G + grp] | ((uint32_t)biases[n * G + grp] << 16);
        }
      }
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* quantizers                                                                */
/* ------------------------------------------------------------------------ */

static int gs_ok(int gs) { return gs == 32 || gs == 64 || gs == 128; }

int orc_quantize(const float* w, int64_t N, int64_t K, int gs, int bits, int mode,
                 uint8_t* codes_out, uint32_t* wq, uint16_t* scales_bf16,
                 uint16_t* biases_bf16, float* scales_f32, float* biases_f32) {
  if (!layout_ok(N, K, bits) || !gs_ok(gs) || K % gs != 0 || (mode != 0 && mode != 1))
    return -1;
  const float nmax = (float)((1 << bits) - 1);
  const float eps = 1e-7f;
  int64_t G = K / gs;
  uint8_t* codes = codes_out;
  if (!codes) {
    codes = (uint8_t*)malloc((size_t)(N * K));
    if (!codes) return -1;
  }
  for (int64_t n = 0; n < N; ++n)
    for (int64_t g = 0; g < G; ++g) {
      const float* wg = w + n * K + g * gs;
      float mn = wg[0], mx = wg[0];
      for (int i = 1; i < gs; ++i) {
        mn = fminf(mn, wg[i]);
        mx = fmaxf(mx, wg[i]);
      }
      float s, b;
      if (mode == 0) {
        s = (mx - mn) / nmax;
        if (mx == mn) s = eps;
        b = mn;
      } else {
        s = fmaxf((mx - mn) / nmax, eps);
        int side = fabsf(mn) > fabsf(mx);
        s = side ? s : -s;
        float edge = side ? mn : mx;
        float q0 = rintf(edge / s);
        if (q0 != 0.0f) {
          s = edge / q0;
          b = edge;
        } else {
          b = 0.0f;
        }
      }
      for (int i = 0; i < gs; ++i) {
        float q = rintf((wg[i] - b) / s);
        q = fminf(fmaxf(q, 0.0f), nmax);
        codes[n * K + g * gs + i] = (uint8_t)q;
      }
      if (scales_bf16) scales_bf16[n * G + g] = orc_bf16_rne(s);
      if (biases_bf16) biases_bf16[n * G + g] = orc_bf16_rne(b);
      if (scales_f32) scales_f32[n * G + g] = s;
      if (biases_f32) biases_f32[n * G + g] = b;
    }
  int rc = 0;
  if (wq) rc = orc_pack_words(codes, N, K, bits, wq);
  if (!codes_out) free(codes);
  return rc;
}

/* ------------------------------------------------------------------------ */
/* dequantization                                                            */
/* ------------------------------------------------------------------------ */

int orc_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                   int64_t N, int64_t K, int gs, int bits, float* out_f32,
                   uint16_t* out_bf16) {
  if (!layout_ok(N, K, bits) || !gs_ok(gs) || K % gs != 0) return -1;
  int64_t W = K * bits / 32, G = K / gs;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      float s = orc_bf16_to_f32(scales[n * G + k / gs]);
      float b = orc_bf16_to_f32(biases[n * G + k / gs]);
      float v = fmaf((float)code_at(wq + n * W, k, bits), s, b);
      if (out_f32) out_f32[n * K + k] = v;
      if (out_bf16) out_bf16[n * K + k] = orc_bf16_rne(v);
    }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* matmul references                                                         */
/* ------------------------------------------------------------------------ */

static int qmm_args_ok(int64_t M, int64_t K, int64_t N, int gs, int bits) {
  return layout_ok(N, K, bits) && gs_ok(gs) && K % gs == 0 && M >= 0;
}

/* round_w = 0: exact fp64 weights; 1: weights rounded to bf16 through fmaf. */
static int qmm_f64_impl(const uint16_t* x, int64_t M, int64_t K, const uint32_t* wq,
                        const uint16_t* scales, const uint16_t* biases, int64_t N,
                        int gs, int bits, const uint16_t* bias, const int64_t* rows,
                        int64_t nrows, int threads, double* y, int round_w) {
  if (!qmm_args_ok(M, K, N, gs, bits)) return -1;
  if (!rows) nrows = M;
  for (int64_t r = 0; r < nrows; ++r)
    if (rows && (rows[r] < 0 || rows[r] >= M)) return -1;
  int64_t W = K * bits / 32, G = K / gs;
  double* xd = (double*)malloc((size_t)(nrows * K) * sizeof(double));
  if (!xd) return -1;
  for (int64_t r = 0; r < nrows; ++r) {
    int64_t m = rows ? rows[r] : r;
    for (int64_t k = 0; k < K; ++k) xd[r * K + k] = orc_bf16_to_f32(x[m * K + k]);
  }
  int fail = 0;
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
  {
    double* wd = (double*)malloc((size_t)K * sizeof(double));
    if (!wd) {
#pragma omp atomic write
      fail = 1;
    }
#pragma omp for schedule(dynamic, 16)
    for (int64_t n = 0; n < N; ++n) {
      if (!wd) continue;
      const uint32_t* row = wq + n * W;
      for (int64_t g = 0; g < G; ++g) {
        float sf = orc_bf16_to_f32(scales[n * G + g]);
        float bf = orc_bf16_to_f32(biases[n * G + g]);
        for (int64_t k = g * gs; k < (g + 1) * gs; ++k) {
          unsigned q = code_at(row, k, bits);
          if (round_w)
            wd[k] = orc_bf16_to_f32(orc_bf16_rne(fmaf((float)q, sf, bf)));
          else
            wd[k] = (double)sf * (double)q + (double)bf;
        }
      }
      double bn = bias ? (double)orc_bf16_to_f32(bias[n]) : 0.0;
      for (int64_t r = 0; r < nrows; ++r) {
        const double* xr = xd + r * K;
        double acc = 0.0;
#pragma omp simd reduction(+ : acc)
        for (int64_t k = 0; k < K; ++k) acc += xr[k] * wd[k];
        y[r * N + n] = acc + bn;
      }
    }
    free(wd);
  }
  free(xd);
  return fail ? -1 : 0;
}

int orc_qmm_f64(const uint16_t* x, int64_t M, int64_t K, const uint32_t* wq,
                const uint16_t* scales, const uint16_t* biases, int64_t N, int gs,
                int bits, const uint16_t* bias, const int64_t* rows, int64_t nrows,
                int threads, double* y) {
  return qmm_f64_impl(x, M, K, wq, scales, biases, N, gs, bits, bias, rows, nrows, threads,
                      y, 0);
}

int orc_qmm_f64_bf16w(const uint16_t* x, int64_t M, int64_t K, const uint32_t* wq,
                      const uint16_t* scales, const uint16_t* biases, int64_t N, int gs,
                      int bits, const uint16_t* bias, const int64_t* rows,
                      int64_t nrows, int threads, double* y) {
  return qmm_f64_impl(x, M, K, wq, scales, biases, N, gs, bits, bias, rows, nrows, threads,
                      y, 1);
}

/* bf16 arithmetic as a bf16 scalar type does it: compute in fp32, round. */
static inline float bfr(float v) { return orc_bf16_to_f32(orc_bf16_rne(v)); }

int orc_qmm_mlx_cpu(const uint16_t* x, int64_t M, int64_t K, const uint32_t* wq,
                    const uint16_t* scales, const uint16_t* biases, int64_t N, int gs,
                    int bits, int accum, const int64_t* rows, int64_t nrows,
                    int threads, uint16_t* y) {
  if (!qmm_args_ok(M, K, N, gs, bits) || (accum != 0 && accum != 1)) return -1;
  if (!rows) nrows = M;
  for (int64_t r = 0; r < nrows; ++r)
    if (rows && (rows[r] < 0 || rows[r] >= M)) return -1;
  const int64_t W = K * bits / 32, G = K / gs;
  const uint32_t mask = (1u << bits) - 1u;
  /* codes are read from the byte stream: `bits` bits at a time, LSB first,
   * from a 64-bit window refilled from whole little-endian words. */
  for (int64_t r = 0; r < nrows; ++r) {
    const uint16_t* xm = x + (rows ? rows[r] : r) * K;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      const uint32_t* wrow = wq + n * W;
      const uint16_t* sc = scales + n * G;
      const uint16_t* bi = biases + n * G;
      uint64_t window = 0;
      int avail = 0;
      int64_t wi = 0;
      float sum = 0.0f;
      const uint16_t* xl = xm;
      for (int64_t g = 0; g < G; ++g) {
        float s = orc_bf16_to_f32(sc[g]);
        float b = orc_bf16_to_f32(bi[g]);
        for (int i = 0; i < gs; ++i) {
          if (avail < bits) {
            window |= (uint64_t)wrow[wi++] << avail;
            avail += 32;
          }
          float q = (float)(window & mask);
          window >>= bits;
          avail -= bits;
          float xv = orc_bf16_to_f32(*xl++);
          if (accum == 0) {
            float wv = bfr(bfr(s * q) + b);
            sum = bfr(sum + bfr(xv * wv));
          } else {
            sum += xv * (s * q + b);
          }
        }
      }
      y[r * N + n] = orc_bf16_rne(sum);
    }
  }
  return 0;
}

void orc_gelu_tanh_bf16(const uint16_t* in, int64_t n, uint16_t* out) {
  const double c = sqrt(2.0 / 3.14159265358979323846);
  for (int64_t i = 0; i < n; ++i) {
    double v = orc_bf16_to_f32(in[i]);
    double g = 0.5 * v * (1.0 + tanh(c * (v + 0.044715 * v * v * v)));
    out[i] = orc_bf16_rne((float)g);
  }
}
