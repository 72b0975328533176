/*
 * nsmlp_oracle.c -- CPU restatement of next_step_ai's blockwise-sparse NF4 MLP
 * decode path.  TEST INFRASTRUCTURE ONLY: this file is the checker.  Only the
 * tests, the smoke check and the CPU-baseline leg of the benchmark load it; the
 * product library never links, calls or falls back to it.
 *
 * What it restates (paths relative to the reference repository):
 *   - router  : llama3_neuroplastic/experiments/streaming_llama_runtime.py
 *               (RT) :4209-4238 (_compute_sparse_basis_latent) and
 *               :4311-4352 (_route_sparse_mlp), with the precision contract
 *               "exact dot product + bias, rounded once to fp16 (RNE)" and the
 *               selection rule "score descending, index ascending".
 *   - NF4     : the bitsandbytes NF4 format as indexed by RT:5439-5483 and
 *               llama3_neuroplastic/triton_sparse_mlp.py (TSM) :851-911
 *               (row-major flattening, even element in the high nibble, one
 *               absmax per quant block of consecutive elements).
 *   - MLP     : the dequant fallback RT:5433-5492 (fp16 rounding points) and
 *               an fp64 reference of the same closed form.
 *   - quantizer: bitsandbytes==0.49.1 quantize_4bit(nf4) / double quant,
 *               restated from its published algorithm (bitsandbytes is not
 *               present here: parity unpinned at that boundary).
 *
 * The exact router here accumulates in __int128 fixed point with LSB 2^-48,
 * which is an independent algorithm from the GPU's error-free fp64 splitting;
 * agreement between the two is what the parity tests check.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

typedef __int128 i128;
typedef unsigned __int128 u128;

/* ------------------------------------------------------------------ fp16 */

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  uint32_t bits;
  if (e == 0x1F) {
    bits = sign | 0x7F800000u | (m << 13);
  } else if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      /* subnormal: value = m * 2^-24 */
      float v = (float)m * (1.0f / 16777216.0f);
      memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static int msb128(u128 v) {
  uint64_t hi = (uint64_t)(v >> 64);
  if (hi) return 127 - __builtin_clzll(hi);
  uint64_t lo = (uint64_t)v;
  return 63 - __builtin_clzll(lo);
}

/* Round sign * M * 2^E (M > 0) to the nearest fp16, ties to even. */
static uint16_t round_to_f16(int neg, u128 M, int E) {
  uint16_t sign = neg ? 0x8000u : 0u;
  if (M == 0) return sign;
  int msb = msb128(M);
  int X = msb + E; /* floor(log2(value)) */
  if (X > 15) return sign | 0x7C00u;
  int q = (X >= -14) ? (X - 10) : -24; /* quantum exponent */
  int shift = q - E;
  u128 R;
  if (shift <= 0) {
    R = M << (-shift);
  } else if (shift >= 127) {
    R = 0; /* far below the smallest subnormal: rounds to zero */
    return sign;
  } else {
    R = M >> shift;
    u128 rem = M - (R << shift);
    u128 half = (u128)1 << (shift - 1);
    if (rem > half || (rem == half && (R & 1))) R += 1;
  }
  if (q == -24) {
    /* subnormal (R <= 1024; R == 1024 is the smallest normal, same bits) */
    return sign | (uint16_t)R;
  }
  if (R == 2048) {
    R = 1024;
    q += 1;
  }
  int expfield = q + 10 + 15;
  if (expfield >= 31) return sign | 0x7C00u;
  return sign | (uint16_t)(expfield << 10) | (uint16_t)(R - 1024);
}

uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  int neg = (int)(x >> 31);
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) {
    uint16_t sign = neg ? 0x8000u : 0u;
    if (ax > 0x7F800000u) return sign | 0x7E00u | (uint16_t)((ax >> 13) & 0x3FFu);
    return sign | 0x7C00u;
  }
  uint32_t e = ax >> 23;
  uint32_t m = ax & 0x7FFFFFu;
  if (e == 0) return round_to_f16(neg, (u128)m, -149);
  return round_to_f16(neg, (u128)(m | 0x800000u), (int)e - 150);
}

uint16_t orc_f64_to_f16(double d) {
  uint64_t x;
  memcpy(&x, &d, 8);
  int neg = (int)(x >> 63);
  uint64_t ax = x & 0x7FFFFFFFFFFFFFFFull;
  if (ax >= 0x7FF0000000000000ull) {
    uint16_t sign = neg ? 0x8000u : 0u;
    if (ax > 0x7FF0000000000000ull) return sign | 0x7E00u;
    return sign | 0x7C00u;
  }
  uint64_t e = ax >> 52;
  uint64_t m = ax & 0xFFFFFFFFFFFFFull;
  if (e == 0) return round_to_f16(neg, (u128)m, -1074);
  return round_to_f16(neg, (u128)(m | (1ull << 52)), (int)e - 1075);
}

/* Exact fixed point (LSB 2^-48) to fp16, RNE. */
uint16_t orc_fix48_to_f16(int64_t hi, uint64_t lo) {
  i128 v = ((i128)hi << 64) | (i128)lo;
  int neg = v < 0;
  u128 M = neg ? (u128)(-v) : (u128)v;
  return round_to_f16(neg, M, -48);
}

static inline uint16_t f16_bits_is_finite(uint16_t h) { return ((h >> 10) & 0x1F) != 0x1F; }

/* fp16 h = (-1)^neg * m * 2^E */
static inline void f16_decode(uint16_t h, int* neg, uint32_t* m, int* E) {
  uint32_t e = (h >> 10) & 0x1Fu;
  *neg = (h >> 15) & 1;
  *m = (h & 0x3FFu) | (e ? 0x400u : 0u);
  *E = (e ? (int)e : 1) - 25;
}

/* Exact sum_i a[i]*b[i] (+ bias) as __int128 fixed point, LSB 2^-48.
 * Returns 0 on success, -1 if any input is inf/NaN.                       */
static int dot_fix48(const uint16_t* a, int a_abs, const uint16_t* b, long n, const uint16_t* bias, i128* out) {
  i128 acc = 0;
  for (long i = 0; i < n; ++i) {
    uint16_t ha = a[i], hb = b[i];
    if (!f16_bits_is_finite(ha) || !f16_bits_is_finite(hb)) return -1;
    int na, nb, Ea, Eb;
    uint32_t ma, mb;
    f16_decode(ha, &na, &ma, &Ea);
    f16_decode(hb, &nb, &mb, &Eb);
    if (a_abs) na = 0;
    int s = Ea + Eb + 48; /* >= 0 */
    i128 t = (i128)((uint64_t)ma * (uint64_t)mb) << s;
    acc += (na ^ nb) ? -t : t;
  }
  if (bias) {
    uint16_t hc = *bias;
    if (!f16_bits_is_finite(hc)) return -1;
    int nc, Ec;
    uint32_t mc;
    f16_decode(hc, &nc, &mc, &Ec);
    i128 t = (i128)mc << (Ec + 48);
    acc += nc ? -t : t;
  }
  *out = acc;
  return 0;
}

/* Exact dot + bias rounded once to fp16.  Returns fp16 bits (0x7E00 on non-finite input). */
uint16_t orc_dot_exact_f16(const uint16_t* a, const uint16_t* b, long n, const uint16_t* bias) {
  i128 v;
  if (dot_fix48(a, 0, b, n, bias, &v) != 0) return 0x7E00u;
  int neg = v < 0;
  u128 M = neg ? (u128)(-v) : (u128)v;
  return round_to_f16(neg, M, -48);
}

/* Exact dot returned as fixed point (for tests that check the rounding step). */
int orc_dot_exact_fix48(const uint16_t* a, const uint16_t* b, long n, const uint16_t* bias, int64_t* hi, uint64_t* lo) {
  i128 v;
  int rc = dot_fix48(a, 0, b, n, bias, &v);
  *hi = (int64_t)(v >> 64);
  *lo = (uint64_t)v;
  return rc;
}

/* Total order key of an fp16 value (larger value -> larger key); -0 == +0. */
static inline uint32_t f16_order_key(uint16_t h) {
  if (h == 0x8000u) h = 0;
  return (h & 0x8000u) ? (uint32_t)(~h & 0xFFFFu) : (uint32_t)(h | 0x8000u);
}

/* ---------------------------------------------------------------- router */

typedef struct {
  uint32_t key;
  int32_t idx;
} keyidx_t;

static int cmp_keyidx_desc(const void* pa, const void* pb) {
  const keyidx_t* a = (const keyidx_t*)pa;
  const keyidx_t* b = (const keyidx_t*)pb;
  if (a->key != b->key) return a->key > b->key ? -1 : 1;
  return a->idx < b->idx ? -1 : (a->idx > b->idx ? 1 : 0);
}

/*
 * Router for one token (RT:4209-4238, RT:4311-4352).
 *   latent  = fp16(x . enc_w[r] + enc_b[r])                  r < R
 *   if basis_top_k < R: keep the basis_top_k largest |latent| (index-ascending ties)
 *   main path   (legacy_abs == 0): score = max(fp16(latent . score_w[j] + score_b[j]), 0)
 *   legacy path (legacy_abs != 0): score = fp16(|latent| . score_w[j])   (score_w = |score_weight|)
 *   if dbn: score = fp16(score * fp16(dbn[j]))
 *   selection: the k largest scores, ties by lowest index, in (score desc, index asc) order.
 * Returns 0, or -1 on non-finite input.
 */
int orc_route_f16(const uint16_t* x, int H, const uint16_t* enc_w, const uint16_t* enc_b, int R, int basis_top_k,
                  const uint16_t* score_w, const uint16_t* score_b, const float* dbn, int NB, int legacy_abs, int k,
                  uint16_t* latent_out, uint16_t* scores_out, int32_t* sel_out) {
  uint16_t* lat = latent_out;
  for (int r = 0; r < R; ++r) {
    i128 v;
    if (dot_fix48(x, 0, enc_w + (long)r * H, H, enc_b ? enc_b + r : NULL, &v) != 0) return -1;
    int neg = v < 0;
    u128 M = neg ? (u128)(-v) : (u128)v;
    lat[r] = round_to_f16(neg, M, -48);
  }
  int btk = basis_top_k < 1 ? 1 : (basis_top_k > R ? R : basis_top_k);
  if (btk < R) {
    keyidx_t* tmp = (keyidx_t*)malloc(sizeof(keyidx_t) * (size_t)R);
    for (int r = 0; r < R; ++r) {
      tmp[r].key = f16_order_key((uint16_t)(lat[r] & 0x7FFFu));
      tmp[r].idx = r;
    }
    qsort(tmp, (size_t)R, sizeof(keyidx_t), cmp_keyidx_desc);
    uint8_t* keep = (uint8_t*)calloc((size_t)R, 1);
    for (int i = 0; i < btk; ++i) keep[tmp[i].idx] = 1;
    for (int r = 0; r < R; ++r)
      if (!keep[r]) lat[r] = (uint16_t)(lat[r] & 0x8000u); /* latent * 0 keeps the sign of zero */
    free(keep);
    free(tmp);
  }
  for (int j = 0; j < NB; ++j) {
    i128 v;
    const uint16_t* bias = (legacy_abs || !score_b) ? NULL : score_b + j;
    if (dot_fix48(lat, legacy_abs, score_w + (long)j * R, R, bias, &v) != 0) return -1;
    int neg = v < 0;
    u128 M = neg ? (u128)(-v) : (u128)v;
    uint16_t s = round_to_f16(neg, M, -48);
    if (!legacy_abs && (s & 0x8000u)) s = 0; /* clamp_min(0) */
    if (dbn) {
      uint16_t d16 = orc_f32_to_f16(dbn[j]);
      float p = orc_f16_to_f32(s) * orc_f16_to_f32(d16); /* exact in fp32 */
      s = orc_f32_to_f16(p);
    }
    scores_out[j] = s;
  }
  int kk = k < 1 ? 1 : (k > NB ? NB : k);
  keyidx_t* order = (keyidx_t*)malloc(sizeof(keyidx_t) * (size_t)NB);
  for (int j = 0; j < NB; ++j) {
    order[j].key = f16_order_key(scores_out[j]);
    order[j].idx = j;
  }
  qsort(order, (size_t)NB, sizeof(keyidx_t), cmp_keyidx_desc);
  for (int i = 0; i < kk; ++i) sel_out[i] = order[i].idx;
  free(order);
  return 0;
}

/* ------------------------------------------------------------------ NF4 */

/* The 16 NF4 code values (QLoRA normal-float 4-bit; bitsandbytes nf4 map). */
static const float NF4_CODE[16] = {
    -1.0f,
    -0.6961928009986877f,
    -0.5250730514526367f,
    -0.39491748809814453f,
    -0.28444138169288635f,
    -0.18477343022823334f,
    -0.09105003625154495f,
    0.0f,
    0.07958029955625534f,
    0.16093020141124725f,
    0.24611230194568634f,
    0.33791524171829224f,
    0.44070982933044434f,
    0.5626170039176941f,
    0.7229568362236023f,
    1.0f,
};

void orc_nf4_code(float* out16) { memcpy(out16, NF4_CODE, sizeof(NF4_CODE)); }

/* Nearest NF4 code of a normalised value: decision thresholds are the
 * midpoints between consecutive codes, compared with '>' (a value exactly on
 * a midpoint takes the lower code), as in the bitsandbytes decision tree.    */
static inline uint8_t nf4_nearest(float v) {
  uint8_t c = 0;
  for (int i = 0; i < 15; ++i) {
    float mid = (float)(((double)NF4_CODE[i] + (double)NF4_CODE[i + 1]) * 0.5);
    if (v > mid) c = (uint8_t)(i + 1);
  }
  return c;
}

/* Blockwise NF4 quantisation of n consecutive fp32 values (row-major flattening),
 * one absmax per qbs elements; element 2i goes to the high nibble of byte i.
 * A block whose absmax is 0 is stored as code 7 (exact zero).                */
void orc_nf4_quantize(const float* w, long n, int qbs, uint8_t* packed, float* absmax) {
  long nblk = n / qbs;
#pragma omp parallel for schedule(static)
  for (long b = 0; b < nblk; ++b) {
    const float* src = w + b * qbs;
    float amax = 0.0f;
    for (int i = 0; i < qbs; ++i) {
      float a = fabsf(src[i]);
      if (a > amax) amax = a;
    }
    absmax[b] = amax;
    float inv = amax > 0.0f ? 1.0f / amax : 0.0f;
    for (int i = 0; i < qbs; i += 2) {
      uint8_t hi = amax > 0.0f ? nf4_nearest(src[i] * inv) : 7;
      uint8_t lo = amax > 0.0f ? nf4_nearest(src[i + 1] * inv) : 7;
      packed[(b * qbs + i) >> 1] = (uint8_t)((hi << 4) | lo);
    }
  }
}

/* NF4 dequantisation to fp32: w = code[nib] * absmax (one fp32 product).   */
void orc_nf4_dequant_f32(const uint8_t* packed, const float* absmax, long n, int qbs, const float* code, float* out) {
#pragma omp parallel for schedule(static)
  for (long e = 0; e < n; ++e) {
    uint8_t byte = packed[e >> 1];
    uint8_t nib = (e & 1) ? (byte & 0x0F) : (byte >> 4);
    out[e] = code[nib] * absmax[e / qbs];
  }
}

/* bitsandbytes signed dynamic 8-bit map (create_dynamic_map(signed=True,
 * max_exponent_bits=7, total_bits=8)), restated from its published
 * construction, which runs in torch fp32: for exponent i in 0..6 the
 * boundaries b = linspace(0.1, 1, 2^i + 1) in fp32, their midpoints
 * fl32(fl32(b[j] + b[j+1]) / 2) scaled by fl32(10^(i-6)) in fp32, with both
 * signs; plus 0 and 1; sorted ascending (256 values).  fp32 linspace(a, b,
 * n) on the CPU is step = fl32(fl32(b - a) / (n - 1)), the first n/2 points
 * fma(step, j, a) and the rest fma(-step, n - 1 - j, b) (one rounding each). */
static int cmp_float_asc(const void* a, const void* b) {
  float x = *(const float*)a, y = *(const float*)b;
  return x < y ? -1 : (x > y ? 1 : 0);
}

static float linspace_f32(float a, float b, int n, int j) {
  const float step = (b - a) / (float)(n - 1);
  return j < n / 2 ? fmaf(step, (float)j, a) : fmaf(-step, (float)(n - 1 - j), b);
}

void orc_dynamic_map_signed(float* out256) {
  int n = 0;
  for (int i = 0; i < 7; ++i) {
    const int items = (1 << i) + 1;
    const float scale = (float)pow(10.0, (double)(i - 6));  /* the Python float 10**(i-6), as fp32 */
    for (int j = 0; j + 1 < items; ++j) {
      const float b0 = linspace_f32(0.1f, 1.0f, items, j), b1 = linspace_f32(0.1f, 1.0f, items, j + 1);
      const float mean = (b0 + b1) / 2.0f;
      out256[n++] = scale * mean;
      out256[n++] = -scale * mean;
    }
  }
  out256[n++] = 0.0f;
  out256[n++] = 1.0f;
  while (n < 256) out256[n++] = 0.0f;
  qsort(out256, 256, sizeof(float), cmp_float_asc);
}

/* Double quantisation of an fp32 absmax vector (bitsandbytes compress_statistics):
 * offset = mean(absmax); a = absmax - offset; blocks of dq_block (bitsandbytes:
 * 256): absmax2 = max|a|, q = index of the nearest map value to
 * a * fl32(1/absmax2) (ties: lower index).
 * Dequantised absmax = fl32(fl32(map[q] * absmax2) + offset).               */
void orc_double_quant_ex(const float* absmax, long n, const float* map256, long dq_block, float offset, uint8_t* q,
                         float* absmax2) {
  long nb = (n + dq_block - 1) / dq_block;
  for (long b = 0; b < nb; ++b) {
    long lo = b * dq_block, hi = lo + dq_block < n ? lo + dq_block : n;
    float amax = 0.0f;
    for (long i = lo; i < hi; ++i) {
      float a = fabsf(absmax[i] - offset);
      if (a > amax) amax = a;
    }
    absmax2[b] = amax;
    float inv = amax > 0.0f ? 1.0f / amax : 0.0f;
    for (long i = lo; i < hi; ++i) {
      float v = (absmax[i] - offset) * inv;
      int best = 0;
      float bd = fabsf(map256[0] - v);
      for (int c = 1; c < 256; ++c) {
        float d = fabsf(map256[c] - v);
        if (d < bd) {
          bd = d;
          best = c;
        }
      }
      q[i] = (uint8_t)best;
    }
  }
}

void orc_double_quant(const float* absmax, long n, const float* map256, uint8_t* q, float* absmax2, float* offset_out) {
  double s = 0.0;
  for (long i = 0; i < n; ++i) s += absmax[i];
  float offset = (float)(s / (double)n);
  *offset_out = offset;
  orc_double_quant_ex(absmax, n, map256, 256, offset, q, absmax2);
}

void orc_double_dequant_ex(const uint8_t* q, const float* absmax2, float offset, const float* map256, long n,
                           long dq_block, float* out) {
  for (long i = 0; i < n; ++i) {
    volatile float p = map256[q[i]] * absmax2[i / dq_block];
    out[i] = p + offset;
  }
}

void orc_double_dequant(const uint8_t* q, const float* absmax2, float offset, const float* map256, long n, float* out) {
  orc_double_dequant_ex(q, absmax2, offset, map256, n, 256, out);
}

/* ------------------------------------------------------------------- MLP */

static inline double silu64(double g) { return g / (1.0 + exp(-g)); }

/*
 * Blockwise-sparse NF4 MLP over the reference's gathered layouts
 * (RT:4630-4660 gate/up, RT:4491-4511 down, RT:4857-4908 layout):
 *   gate/up packed [A, 32, H/2] u8, absmax [A, 32, H/qbs] f32
 *   down    packed [H, A, 16]  u8, absmax [H, A]        f32
 *   x [rows, H] fp16; active_local [rows, kk] int32 (slot in 0..A-1, -1 = none)
 * flat_mask semantics: row t only uses its own slots (RT:5453).
 *   y_exact    : fp64 closed form y = sum_b Wd[:,b] (silu(Wg_b x) * (Wu_b x))
 *   y_fallback : fp16 rounding points of the dequant fallback (RT:5439-5488):
 *                Wg = f16(code*absmax); g = f16(sum Wg x); a = f16(f16(silu(g)) * u);
 *                Wd = f16(f16(code) * f16(absmax)); y = f16(sum Wd a).
 *   Either output pointer may be NULL.  Sums are accumulated in fp64.
 */
int orc_sparse_mlp(int rows, int H, int A, int qbs, const uint16_t* x, const int32_t* active_local, int kk,
                   const uint8_t* gate_packed, const float* gate_absmax, const uint8_t* up_packed,
                   const float* up_absmax, const uint8_t* down_packed, const float* down_absmax, const float* code,
                   double* y_exact, uint16_t* y_fallback, double* a_exact_out) {
  const int want_exact = y_exact != NULL || a_exact_out != NULL;
  const int want_fb = y_fallback != NULL;
  const int BS = 32;
  if (H % qbs != 0 || qbs % 2 != 0) return -1;
  const long row_bytes = H / 2;
  const long row_abs = H / qbs;
  double* xf = (double*)malloc(sizeof(double) * (size_t)H);
  double* a_ex = (double*)malloc(sizeof(double) * (size_t)A * BS);
  uint16_t* a16 = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)A * BS);
  uint8_t* use = (uint8_t*)malloc((size_t)A);
  uint16_t code16[16];
  for (int i = 0; i < 16; ++i) code16[i] = orc_f32_to_f16(code[i]);
  for (int t = 0; t < rows; ++t) {
    const uint16_t* xt = x + (long)t * H;
    for (int c = 0; c < H; ++c) xf[c] = (double)orc_f16_to_f32(xt[c]);
    memset(use, 0, (size_t)A);
    for (int i = 0; i < kk; ++i) {
      int s = active_local[(long)t * kk + i];
      if (s >= 0 && s < A) use[s] = 1;
    }
#pragma omp parallel for schedule(dynamic, 1)
    for (int blk = 0; blk < A; ++blk) {
      for (int r = 0; r < BS; ++r) {
        long o = (long)blk * BS + r;
        if (!use[blk]) {
          a_ex[o] = 0.0;
          a16[o] = 0;
          continue;
        }
        double ge = 0.0, ue = 0.0, gf = 0.0, uf = 0.0;
        const uint8_t* gp = gate_packed + o * row_bytes;
        const uint8_t* upp = up_packed + o * row_bytes;
        const float* ga = gate_absmax + o * row_abs;
        const float* ua = up_absmax + o * row_abs;
        for (int c = 0; c < H; ++c) {
          uint8_t gb = gp[c >> 1], ub = upp[c >> 1];
          int gn = (c & 1) ? (gb & 0xF) : (gb >> 4);
          int un = (c & 1) ? (ub & 0xF) : (ub >> 4);
          float gs = ga[c / qbs], us = ua[c / qbs];
          if (want_exact) {
            ge += (double)code[gn] * (double)gs * xf[c];
            ue += (double)code[un] * (double)us * xf[c];
          }
          if (want_fb) {
            gf += (double)orc_f16_to_f32(orc_f32_to_f16(code[gn] * gs)) * xf[c];
            uf += (double)orc_f16_to_f32(orc_f32_to_f16(code[un] * us)) * xf[c];
          }
        }
        a_ex[o] = silu64(ge) * ue;
        if (want_fb) {
          uint16_t g16 = orc_f64_to_f16(gf), u16 = orc_f64_to_f16(uf);
          uint16_t s16 = orc_f64_to_f16(silu64((double)orc_f16_to_f32(g16)));
          a16[o] = orc_f32_to_f16(orc_f16_to_f32(s16) * orc_f16_to_f32(u16));
        }
      }
    }
    if (a_exact_out) memcpy(a_exact_out + (long)t * A * BS, a_ex, sizeof(double) * (size_t)A * BS);
#pragma omp parallel for schedule(static)
    for (int o = 0; o < H; ++o) {
      double ye = 0.0, yf = 0.0;
      for (int blk = 0; blk < A; ++blk) {
        if (!use[blk]) continue;
        const uint8_t* dp = down_packed + ((long)o * A + blk) * (BS / 2);
        float dabs = down_absmax[(long)o * A + blk];
        uint16_t dabs16 = orc_f32_to_f16(dabs);
        for (int j = 0; j < BS; ++j) {
          uint8_t b = dp[j >> 1];
          int n = (j & 1) ? (b & 0xF) : (b >> 4);
          long ai = (long)blk * BS + j;
          if (want_exact) ye += (double)code[n] * (double)dabs * a_ex[ai];
          if (want_fb) {
            float wd = orc_f16_to_f32(code16[n]) * orc_f16_to_f32(dabs16);
            yf += (double)orc_f16_to_f32(orc_f32_to_f16(wd)) * (double)orc_f16_to_f32(a16[ai]);
          }
        }
      }
      if (y_exact) y_exact[(long)t * H + o] = ye;
      if (y_fallback) y_fallback[(long)t * H + o] = orc_f64_to_f16(yf);
    }
  }
  free(xf);
  free(a_ex);
  free(a16);
  free(use);
  return 0;
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ------------------------------------------------------ array conversions */

void orc_f32_to_f16_array(const float* in, long n, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) out[i] = orc_f32_to_f16(in[i]);
}

void orc_f16_to_f32_array(const uint16_t* in, long n, float* out) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) out[i] = orc_f16_to_f32(in[i]);
}

void orc_f64_to_f16_array(const double* in, long n, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) out[i] = orc_f64_to_f16(in[i]);
}
