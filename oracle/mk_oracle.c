/*
 * CPU oracle for the batch-small decode step (TEST INFRASTRUCTURE ONLY).
 *
 * This file is a checker: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product (the HIP library) never calls it.
 *
 * It restates the reference's CPU numerical reference, examples/llm/ref_numpy.py (Ref.step,
 * :105-158), with bf16 round-to-nearest-even at exactly the points that file rounds (bfr, :26-32).
 * Where the reference leaves the fp32 evaluation order to numpy/BLAS (matvec `@`, np.mean, .sum()),
 * this oracle fixes one documented order, the same order the gfx950 kernels use, so that GPU
 * results can be compared bit for bit:
 *
 *   dot64(w, x, K)   64 interleaved fp32 accumulators, acc[k % 64] = fma(w[k], x[k], acc[k % 64]) for
 *                    k ascending, then the lane reduction of lanes_reduce() below (quad swaps, 8- and 16-lane
 *                    mirrors, rows combined pairwise).  Every matvec and every sum of squares uses it.
 *   attention        chunks of 64 positions; per chunk the local max m_c, p_t = expf(s_t - m_c),
 *                    l_c and a_c[d] as ascending-t fma chains; chunks merged in ascending order with
 *                    w_c = expf(m_c - M):  L = fma(w_c, l_c, L), A[d] = fma(w_c, a_c[d], A[d]); o = bfr(A / L).
 *                    This is the split/merge form of the reference's GPU tiles (examples/llm/tiles.hip:175-247),
 *                    mathematically the softmax of ref_numpy.py:122-129.
 *   softmax sums     over experts: the dot64 accumulator pattern with plain adds.
 *   exp              mk_expf below: Cody-Waite reduction by ln2 and a degree-7 Taylor polynomial.
 *   DeepSeek-V2      (arch 1) the absorbed multi-head latent attention, yarn RoPE with the
 *                    DeepSeek interleave, fp32 router with unnormalised top-k, shared experts and leading dense layers
 *                    of the reference's MLA decode specification
 *                    (examples/dsv2lite/results/2026-10-14-k1/b_alld4r0l1kvs_stamps/fleet_src/host/reference_decode.py,
 *                    a third-party snapshot the reference keeps: :78-118 yarn, :120-136 RoPE, :210-256 attention,
 *                    :259-291 MLP and MoE, :294-302 layer), with the fixed orders of mla_layer_step below.
 *   fp8 weights      (wdtype 1) the QKV, O, expert and dense MLP matrices are held as OCP
 *                    e4m3 with one fp32 scale per output row, quantised from the seeded bf16 rows: s = amax / 448,
 *                    q = e4m3(w / s) rounded to nearest even and saturated at +-448.  A matvec row is
 *                    dot64(e4m3 values, x) * s, followed by the bf16 path's rounding points.  wdtype 2 (oracle
 *                    only) dequantises instead, w' = bfr(e4m3(q) * s), into the bf16 dot: the HF-style reference
 *                    the reference's fp8 fixtures build (examples/glm53/cpu_check.py:93-98), for the 5e-2 gate.
 *
 * The seeded weight generator (splitmix64 counter stream + Box-Muller with polynomial log/sin/cos, all
 * in IEEE basic operations) is specified here independently of the device code that must reproduce it.
 *
 * Compile: gcc -O3 -mavx2 -mfma -ffp-contract=off -fopenmp -shared -fPIC (see oracle/Makefile).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>
#include <immintrin.h>

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------ bf16 */
/* ref_numpy.py:26-32 bfr(): u + 0x7FFF + lsb, masked to the top 16 bits */
static inline float bfr(float x) {
  uint32_t u; memcpy(&u, &x, 4);
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  float r; memcpy(&r, &u, 4); return r;
}
static inline uint16_t f2bf(float x) {
  uint32_t u; memcpy(&u, &x, 4);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
static inline float bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16; float r; memcpy(&r, &u, 4); return r;
}

/* ------------------------------------------------------------------ exp */
/* exp(x) in IEEE single operations only: n = floor(x*log2e + 1/2), r = x - n*ln2 (Cody-Waite, two
 * constants), e^r by a degree-7 Taylor polynomial in Horner form with fma, times 2^n applied in two
 * exact halves.  Results below 2^-125 are returned as 0 (no subnormal outputs); x > 88.72283 gives inf. */
static inline float mk_expf(float x) {
  if (!(x > -87.0f)) return (x != x) ? x : 0.0f;
  if (x > 88.72283f) return INFINITY;
  const float n = floorf(fmaf(x, 1.44269504f, 0.5f));
  float r = fmaf(n, -0.693359375f, x);
  r = fmaf(n, 2.12194440e-4f, r);
  float p = 1.98412698e-4f;                 /* 1/5040 */
  p = fmaf(p, r, 1.38888889e-3f);           /* 1/720  */
  p = fmaf(p, r, 8.33333333e-3f);           /* 1/120  */
  p = fmaf(p, r, 4.16666667e-2f);           /* 1/24   */
  p = fmaf(p, r, 1.66666667e-1f);           /* 1/6    */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n, h = ni / 2, g = ni - h;
  uint32_t b1 = (uint32_t)(h + 127) << 23, b2 = (uint32_t)(g + 127) << 23;
  float s1, s2; memcpy(&s1, &b1, 4); memcpy(&s2, &b2, 4);
  return (p * s1) * s2;
}

/* ------------------------------------------------------------------ seeded generator */
/* splitmix64 (Steele, Lea, Flood 2014): output i of the stream with state `key` is mix(key + (i+1)*gamma). */
static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
static inline uint64_t stream_key(uint64_t seed, uint64_t stream) { return mix64(mix64(seed) ^ stream); }
static inline uint64_t stream_bits(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull); }

/* ln(u), u in (0, 1]: u = m * 2^e with m in [sqrt(1/2), sqrt(2)), ln m = 2 atanh(s), s = (m-1)/(m+1). */
static inline float mk_logf(float u) {
  uint32_t b; memcpy(&b, &u, 4);
  int e = (int)((b >> 23) & 0xFF) - 127;
  uint32_t mb = (b & 0x007FFFFFu) | 0x3F800000u;
  float m; memcpy(&m, &mb, 4);
  if (m > 1.41421356f) { m = m * 0.5f; e += 1; }
  const float s = (m - 1.0f) / (m + 1.0f), s2 = s * s;
  float p = 7.69230769e-2f;                 /* 1/13 */
  p = fmaf(p, s2, 9.09090909e-2f);          /* 1/11 */
  p = fmaf(p, s2, 1.11111111e-1f);          /* 1/9  */
  p = fmaf(p, s2, 1.42857143e-1f);          /* 1/7  */
  p = fmaf(p, s2, 2.00000000e-1f);          /* 1/5  */
  p = fmaf(p, s2, 3.33333333e-1f);          /* 1/3  */
  p = fmaf(p, s2, 1.0f);
  const float lnm = 2.0f * s * p;
  const float fe = (float)e;
  return fmaf(fe, 0.693145752f, fmaf(fe, 1.42860677e-6f, lnm));
}
/* sin and cos of phi in [0, pi/2) by Taylor polynomials (degrees 13 and 14) in Horner form with fma. */
static inline void mk_sincos_q(float phi, float* s, float* c) {
  const float x2 = phi * phi;
  float ps = 1.60590438e-10f;               /*  1/13! */
  ps = fmaf(ps, x2, -2.50521084e-8f);       /* -1/11! */
  ps = fmaf(ps, x2, 2.75573192e-6f);        /*  1/9!  */
  ps = fmaf(ps, x2, -1.98412698e-4f);       /* -1/7!  */
  ps = fmaf(ps, x2, 8.33333333e-3f);        /*  1/5!  */
  ps = fmaf(ps, x2, -1.66666667e-1f);       /* -1/3!  */
  ps = fmaf(ps, x2, 1.0f);
  *s = phi * ps;
  float pc = -1.14707456e-11f;              /* -1/14! */
  pc = fmaf(pc, x2, 2.08767570e-9f);        /*  1/12! */
  pc = fmaf(pc, x2, -2.75573192e-7f);       /* -1/10! */
  pc = fmaf(pc, x2, 2.48015873e-5f);        /*  1/8!  */
  pc = fmaf(pc, x2, -1.38888889e-3f);       /* -1/6!  */
  pc = fmaf(pc, x2, 4.16666667e-2f);        /*  1/4!  */
  pc = fmaf(pc, x2, -0.5f);                 /* -1/2!  */
  pc = fmaf(pc, x2, 1.0f);
  *c = pc;
}
/* standard normal for element i of a stream: pair i/2 gives (r cos t, r sin t) by Box-Muller. */
static inline float mk_normal(uint64_t key, uint64_t i) {
  const uint64_t bits = stream_bits(key, i >> 1);
  const uint32_t a = (uint32_t)(bits >> 40), b = (uint32_t)((bits >> 16) & 0xFFFFFFu);
  const float u1 = (float)(a + 1u) * 5.96046448e-8f;          /* 2^-24 */
  const float r = sqrtf(-2.0f * mk_logf(u1));
  const uint32_t q = b >> 22;
  const float phi = (float)(b & 0x3FFFFFu) * 2.38418579e-7f * 1.57079637f;   /* 2^-22 * pi/2 */
  float s, c; mk_sincos_q(phi, &s, &c);
  float cs, sn;
  switch (q) { case 0: cs = c; sn = s; break; case 1: cs = -s; sn = c; break;
               case 2: cs = -c; sn = -s; break; default: cs = s; sn = -c; break; }
  return r * ((i & 1) ? sn : cs);
}

EXPORT uint64_t orc_splitmix64(uint64_t state, uint64_t i) { return stream_bits(state, i); }
EXPORT uint64_t orc_stream_key(uint64_t seed, uint64_t stream) { return stream_key(seed, stream); }
EXPORT float orc_expf(float x) { return mk_expf(x); }
EXPORT float orc_logf(float x) { return mk_logf(x); }
EXPORT void orc_sincos_q(float phi, float* s, float* c) { mk_sincos_q(phi, s, c); }

/* n values of stream `stream` starting at element `start`, bf16(scale * z) (natural element order). */
EXPORT void orc_gen_normal_bf16(uint64_t seed, uint64_t stream, uint64_t start, uint64_t n, float scale, uint16_t* out) {
  const uint64_t key = stream_key(seed, stream);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)n; ++i) out[i] = f2bf(scale * mk_normal(key, start + (uint64_t)i));
}
EXPORT void orc_gen_normal_f32(uint64_t seed, uint64_t stream, uint64_t start, uint64_t n, float* out) {
  const uint64_t key = stream_key(seed, stream);
  for (uint64_t i = 0; i < n; ++i) out[i] = mk_normal(key, start + i);
}
/* uniform integers in [0, bound): (top 32 bits * bound) >> 32 */
EXPORT void orc_gen_tokens(uint64_t seed, uint64_t stream, uint64_t n, uint32_t bound, int32_t* out) {
  const uint64_t key = stream_key(seed, stream);
  for (uint64_t i = 0; i < n; ++i) out[i] = (int32_t)(((stream_bits(key, i) >> 32) * (uint64_t)bound) >> 32);
}

/* ------------------------------------------------------------------ reductions */
/* The lane reduction of a wave64, in the order the gfx950 kernels combine lanes: partner l^1, then l^2 (both within
 * a quad), then the mirror inside 8 lanes (l <-> 7-l), then the mirror inside 16 lanes (l <-> 15-l); after that
 * each 16-lane row holds its row sum in every lane, and the rows are combined as (row0 + row1) + (row2 + row3). */
static inline float lanes_reduce(float* a) {
  float t[64];
  for (int l = 0; l < 64; ++l) t[l] = a[l] + a[l ^ 1];
  for (int l = 0; l < 64; ++l) a[l] = t[l] + t[l ^ 2];
  for (int l = 0; l < 64; ++l) t[l] = a[l] + a[(l & ~7) | (7 - (l & 7))];
  for (int l = 0; l < 64; ++l) a[l] = t[l] + t[(l & ~15) | (15 - (l & 15))];
  return (a[0] + a[16]) + (a[32] + a[48]);
}
#define butterfly64 lanes_reduce
/* canonical dot: w bf16, x fp32 (bf16-valued in every use), K a multiple of 64 */
static inline float dot64(const uint16_t* w, const float* x, int K) {
  float acc[64];
  for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
  for (int k0 = 0; k0 < K; k0 += 64)
    for (int l = 0; l < 64; ++l) acc[l] = fmaf(bf2f(w[k0 + l]), x[k0 + l], acc[l]);
  return butterfly64(acc);
}
static inline float sumsq64(const float* x, int K) {
  float acc[64];
  for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
  for (int k0 = 0; k0 < K; k0 += 64)
    for (int l = 0; l < 64; ++l) acc[l] = fmaf(x[k0 + l], x[k0 + l], acc[l]);
  return butterfly64(acc);
}
/* sum over n values in the same 64-lane pattern with plain adds (n need not be a multiple of 64) */
static inline float sum64(const float* v, int n) {
  float acc[64];
  for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
  for (int k = 0; k < n; ++k) acc[k & 63] = acc[k & 63] + v[k];
  return butterfly64(acc);
}
EXPORT float orc_dot64(const uint16_t* w, const float* x, int K) { return dot64(w, x, K); }

/* ------------------------------------------------------------------ fp8 e4m3 (OCP "fn": no infinities, max 448) */
/* code s.eeee.mmm: e = 0 subnormal m * 2^-9, else (1 + m/8) * 2^(e-7); 0x7F / 0xFF are NaN (never produced here) */
static inline float e4m3_to_f32(uint8_t c) {
  const int e = (c >> 3) & 15, mt = c & 7;
  const float v = e == 0 ? ldexpf((float)mt, -9) : ldexpf(1.0f + (float)mt / 8.0f, e - 7);
  return (c & 0x80) ? -v : v;
}
/* round to nearest even, saturating: |f| >= 448 (or inf) -> 448; below 2^-6 the subnormal grid of 2^-9 */
static inline uint8_t f32_to_e4m3(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80);
  const uint32_t a = u & 0x7FFFFFFFu;
  float af;
  memcpy(&af, &a, 4);
  if (af != af) return (uint8_t)(sign | 0x7E);              /* NaN input: never produced by quantize_rows */
  if (af >= 448.0f) return (uint8_t)(sign | 0x7E);
  if (af < 0.015625f) return (uint8_t)(sign | (uint8_t)rintf(af * 512.0f));   /* exact scaling, then RNE */
  int e = (int)(a >> 23) - 127;                              /* -6 .. 8 */
  uint32_t qm = (a >> 20) & 7, rem = a & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (qm & 1))) ++qm;
  if (qm == 8) { qm = 0; ++e; }
  if (e > 8 || (e == 8 && qm > 6)) return (uint8_t)(sign | 0x7E);
  return (uint8_t)(sign | (uint8_t)((e + 7) << 3) | (uint8_t)qm);
}
EXPORT float orc_e4m3_to_f32(uint8_t c) { return e4m3_to_f32(c); }
/* the 256 decoded values, filled from e4m3_to_f32 when the library loads (the dot loops read them from here) */
static float e4m3_lut[256];
static void __attribute__((constructor)) fill_e4m3_lut(void) {
  for (int c = 0; c < 256; ++c) e4m3_lut[c] = e4m3_to_f32((uint8_t)c);
}
static inline float e4m3_f(uint8_t c) { return e4m3_lut[c]; }
EXPORT uint8_t orc_f32_to_e4m3(float f) { return f32_to_e4m3(f); }

/* per-row quantisation of R rows of K bf16 values */
static void quantize_rows(const uint16_t* w, size_t R, int K, uint8_t* q, float* sc) {
#pragma omp parallel for schedule(static)
  for (size_t r = 0; r < R; ++r) {
    float amax = 0.0f;
    for (int k = 0; k < K; ++k) { const float v = fabsf(bf2f(w[r * K + k])); if (v > amax) amax = v; }
    const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
    sc[r] = s;
    for (int k = 0; k < K; ++k) q[r * K + k] = f32_to_e4m3(bf2f(w[r * K + k]) / s);
  }
}
EXPORT void orc_quantize_rows(const uint16_t* w, int64_t R, int K, uint8_t* q, float* sc) { quantize_rows(w, (size_t)R, K, q, sc); }

/* canonical dot over e4m3 values (exact in fp32) */
static inline float dot64_q(const uint8_t* q, const float* x, int K) {
  float acc[64];
  for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
  for (int k0 = 0; k0 < K; k0 += 64)
    for (int l = 0; l < 64; ++l) acc[l] = fmaf(e4m3_f(q[k0 + l]), x[k0 + l], acc[l]);
  return butterfly64(acc);
}
/* canonical dot over dequantised bf16 weights bfr(e4m3 * s) (wdtype 2) */
static inline float dot64_deq(const uint8_t* q, float s, const float* x, int K) {
  float acc[64];
  for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
  for (int k0 = 0; k0 < K; k0 += 64)
    for (int l = 0; l < 64; ++l) acc[l] = fmaf(bfr(e4m3_f(q[k0 + l]) * s), x[k0 + l], acc[l]);
  return butterfly64(acc);
}
EXPORT float orc_dot64_q(const uint8_t* q, const float* x, int K) { return dot64_q(q, x, K); }
EXPORT float orc_sum64(const float* v, int n) { return sum64(v, n); }

/* ------------------------------------------------------------------ model pieces */
/* ref_numpy.py:71-73 rmsnorm: r = 1/sqrt(mean(x^2) + eps); out = bfr(w * bfr(x * r)) */
static void rmsnorm(const float* x, const uint16_t* w, int n, float eps, float* out) {
  const float ss = sumsq64(x, n);
  const float r = 1.0f / sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; ++i) out[i] = bfr((w ? bf2f(w[i]) : 1.0f) * bfr(x[i] * r));
}
EXPORT void orc_rmsnorm(const float* x, const uint16_t* w, int n, float eps, float* out) { rmsnorm(x, w, n, eps, out); }

/* ref_numpy.py:76-81 rope_tables: inv = 1/theta^(2i/hd), f = pos*inv (fp32), bf16(cos f), bf16(sin f) */
EXPORT void orc_rope_tables(float theta, int hd, int ctx, float* cos_out, float* sin_out) {
  const int half = hd / 2;
  for (int i = 0; i < half; ++i) {
    const float inv = 1.0f / powf(theta, (float)(2 * i) / (float)hd);
    for (int p = 0; p < ctx; ++p) {
      const float f = (float)p * inv;
      cos_out[(size_t)p * half + i] = bfr(cosf(f));
      sin_out[(size_t)p * half + i] = bfr(sinf(f));
    }
  }
}
/* ref_numpy.py:84-88 apply_rope (rotate_half): bfr(bfr(v*c) + bfr(rot*s)) */
static void apply_rope(float* v, int hd, const float* cs, const float* sn) {
  const int half = hd / 2;
  float t[512];
  for (int d = 0; d < hd; ++d) {
    const int i = d < half ? d : d - half;
    const float rot = d < half ? -v[d + half] : v[d - half];
    t[d] = bfr(bfr(v[d] * cs[i]) + bfr(rot * sn[i]));
  }
  memcpy(v, t, sizeof(float) * (size_t)hd);
}
EXPORT void orc_apply_rope(float* v, int hd, const float* cs, const float* sn) { apply_rope(v, hd, cs, sn); }

/* ref_numpy.py:91-92 silu */
static inline float silu(float g) { return g / (1.0f + mk_expf(-g)); }
EXPORT float orc_silu(float g) { return silu(g); }

/* paged KV addressing (etx/ops/attnprep.py:146-168; etx/importer/spec.py:274-281):
 * K [block][NKV][HD/8][BS][8], V [block][NKV][HD][BS]; physical block = block_table[pos / BS]. */
static inline size_t kv_k_index(int blk, int off, int h, int d, int NKV, int HD, int BS) {
  return ((((size_t)blk * NKV + h) * (HD / 8) + d / 8) * BS + off) * 8 + d % 8;
}
static inline size_t kv_v_index(int blk, int off, int h, int d, int NKV, int HD, int BS) {
  return (((size_t)blk * NKV + h) * HD + d) * BS + off;
}
EXPORT int64_t orc_kv_k_index(int blk, int off, int h, int d, int NKV, int HD, int BS) { return (int64_t)kv_k_index(blk, off, h, d, NKV, HD, BS); }
EXPORT int64_t orc_kv_v_index(int blk, int off, int h, int d, int NKV, int HD, int BS) { return (int64_t)kv_v_index(blk, off, h, d, NKV, HD, BS); }

#define ATT_CHUNK 64
/* one q head over positions 0..n-1 of kv head `h` (ref_numpy.py:122-129 in the chunked order above).
 * `q` is bf16-valued fp32 [HD]; the scale is fp32(1/sqrt(HD)) applied after the dot, as the reference does. */
static void attention_head(const float* q, const uint16_t* kc, const uint16_t* vc, const int32_t* btab,
                           int n, int h, int NKV, int HD, int BS, float* o) {
  const float scale = (float)(1.0 / sqrt((double)HD));
  float A[512], a[512];
  float L = 0.0f, M = -INFINITY;
  const int nch = (n + ATT_CHUNK - 1) / ATT_CHUNK;
  float mc[256];                                                 /* chunks: n <= 16384 positions */
  for (int c = 0; c < nch; ++c) {
    const int t0 = c * ATT_CHUNK, t1 = t0 + ATT_CHUNK < n ? t0 + ATT_CHUNK : n;
    float m = -INFINITY;
    for (int t = t0; t < t1; ++t) {
      const int blk = btab[t / BS], off = t % BS;
      float s = 0.0f;
      for (int d = 0; d < HD; ++d) s = fmaf(q[d], bf2f(kc[kv_k_index(blk, off, h, d, NKV, HD, BS)]), s);
      s = s * scale;
      if (s > m) m = s;
    }
    mc[c] = m;
    if (m > M) M = m;
  }
  for (int d = 0; d < HD; ++d) A[d] = 0.0f;
  for (int c = 0; c < nch; ++c) {
    const int t0 = c * ATT_CHUNK, t1 = t0 + ATT_CHUNK < n ? t0 + ATT_CHUNK : n;
    float l = 0.0f;
    for (int d = 0; d < HD; ++d) a[d] = 0.0f;
    for (int t = t0; t < t1; ++t) {
      const int blk = btab[t / BS], off = t % BS;
      float s = 0.0f;
      for (int d = 0; d < HD; ++d) s = fmaf(q[d], bf2f(kc[kv_k_index(blk, off, h, d, NKV, HD, BS)]), s);
      s = s * scale;
      const float p = mk_expf(s - mc[c]);
      l = l + p;
      for (int d = 0; d < HD; ++d) a[d] = fmaf(p, bf2f(vc[kv_v_index(blk, off, h, d, NKV, HD, BS)]), a[d]);
    }
    const float w = mk_expf(mc[c] - M);
    L = fmaf(w, l, L);
    for (int d = 0; d < HD; ++d) A[d] = fmaf(w, a[d], A[d]);
  }
  for (int d = 0; d < HD; ++d) o[d] = bfr(A[d] / L);
}
EXPORT void orc_attention_head(const float* q, const uint16_t* kc, const uint16_t* vc, const int32_t* btab,
                               int n, int h, int NKV, int HD, int BS, float* o) {
  attention_head(q, kc, vc, btab, n, h, NKV, HD, BS, o);
}

/* ref_numpy.py:135-140: fp32 softmax over E logits, top-k by probability with ties to the lower id,
 * optional renormalisation (selection-order sum), bf16 weights. */
static void route(const float* logits, int E, int K, int renorm, int32_t* ids, float* wts) {
  float M = -INFINITY;
  for (int e = 0; e < E; ++e) if (logits[e] > M) M = logits[e];
  float p[1024];
  for (int e = 0; e < E; ++e) p[e] = mk_expf(logits[e] - M);
  const float S = sum64(p, E);
  for (int e = 0; e < E; ++e) p[e] = p[e] / S;
  unsigned char taken[1024] = {0};
  float sel = 0.0f, wv[64];
  for (int k = 0; k < K; ++k) {
    int bi = -1; float bv = -1.0f;
    for (int e = 0; e < E; ++e) if (!taken[e] && p[e] > bv) { bv = p[e]; bi = e; }
    taken[bi] = 1; ids[k] = bi; wv[k] = bv; sel = sel + bv;
  }
  for (int k = 0; k < K; ++k) wts[k] = bfr(renorm ? wv[k] / sel : wv[k]);
}
EXPORT void orc_route(const float* logits, int E, int K, int renorm, int32_t* ids, float* wts) { route(logits, E, K, renorm, ids, wts); }

/* ------------------------------------------------------------------ model */
typedef struct {
  int32_t H, NH, NKV, HD, I, E, TOPK, MI, L, V;
  int32_t moe, qk_norm, norm_topk, block_size, max_ctx, batch;
  float eps, theta;
  int32_t wdtype;                 /* 0 bf16 weights; 1 fp8 e4m3 + per-row scales; 2 fp8 dequantised to bf16 */
  int32_t arch;                   /* 0 Qwen3; 1 DeepSeek-V2 (MLA, shared experts, leading dense layers) */
  int32_t kv_lora, qk_nope, qk_rope, v_head;
  int32_t n_shared, first_dense, dense_I;
  float routed_scale, rope_factor, rope_mscale, rope_mscale_all, beta_fast, beta_slow;
  int32_t rope_orig_max;
} orc_config;

/* tensor streams of the seeded generator: kind << 48 | (layer + 1) << 24 | expert */
enum { S_EMBED = 1, S_LMHEAD = 2, S_WQKV = 3, S_WO = 4, S_ROUTER = 5, S_W13 = 6, S_W2 = 7, S_WGU = 8, S_WD = 9,
       S_KINIT = 10, S_VINIT = 11, S_XIN = 12, S_PROMPT = 13, S_WKVB = 14, S_WSGU = 15, S_WSD = 16 };
static inline uint64_t sid(int kind, int layer, int expert) {
  return ((uint64_t)kind << 48) | ((uint64_t)(layer + 1) << 24) | (uint64_t)expert;
}
EXPORT uint64_t orc_stream_id(int kind, int layer, int expert) { return sid(kind, layer, expert); }

/* a weight matrix: bf16 rows (w), or e4m3 rows (q) with one fp32 scale per row (s) */
typedef struct {
  uint16_t* w;
  uint8_t* q;
  float* s;
} orc_mat;

typedef struct {
  orc_mat wqkv, wo, wgu, wd;      /* DeepSeek-V2: wqkv = [q_proj; kv_a_proj_with_mqa] */
  uint16_t* wr;                   /* the router stays bf16 */
  orc_mat *w13, *w2;              /* per expert, generated on first use */
  uint16_t* wkvb;                 /* DeepSeek-V2 kv_b_proj [NH * (qk_nope + v_head)][kv_lora] */
  orc_mat wsgu, wsd;              /* DeepSeek-V2 shared experts: gate/up interleaved, down */
  uint16_t *kc, *vc;              /* DeepSeek-V2: kc is the latent cache [blk][(kv_lora + qk_rope)/8][BS][8] */
} orc_layer;

typedef struct {
  orc_config c;
  uint64_t seed;
  uint16_t *embed, *lm_head;
  orc_layer* ly;
  int32_t* btab;                  /* [batch][nbps]: sequence b's logical block i -> physical block */
  int nblocks, nbps, batch;
  float *rcos, *rsin;             /* DeepSeek-V2: fp32 yarn tables [max_ctx][qk_rope / 2] */
  float scale;
  float attn_scale;
  int mfma;                       /* QKV, O, router, expert gate/up and down and lm_head rows in the matrix-core
                                     orders (batched kernels of capacity >= 8) */
} orc_model;

static uint16_t* gen_tensor(uint64_t seed, uint64_t stream, size_t n, float scale) {
  uint16_t* p = (uint16_t*)malloc(n * sizeof(uint16_t));
  if (p) orc_gen_normal_bf16(seed, stream, 0, n, scale, p);
  return p;
}
/* a seeded R x K matrix, quantised (and its bf16 rows dropped) when the model's weights are fp8 */
static orc_mat gen_mat(uint64_t seed, uint64_t stream, size_t R, int K, float scale, int wdtype) {
  orc_mat m = {gen_tensor(seed, stream, R * (size_t)K, scale), NULL, NULL};
  if (wdtype && m.w) {
    m.q = (uint8_t*)malloc(R * (size_t)K);
    m.s = (float*)malloc(R * sizeof(float));
    quantize_rows(m.w, R, K, m.q, m.s);
    free(m.w);
    m.w = NULL;
  }
  return m;
}
static void free_mat(orc_mat* m) { free(m->w); free(m->q); free(m->s); }
/* row r of a matrix dotted with x (the matvec value before its bf16 rounding) */
static inline float mat_dot(const orc_mat* m, int wdtype, size_t r, const float* x, int K) {
  if (wdtype == 0) return dot64(m->w + r * K, x, K);
  if (wdtype == 1) return dot64_q(m->q + r * K, x, K) * m->s[r];
  return dot64_deq(m->q + r * K, m->s[r], x, K);
}

static void* mla_model_create(orc_model* m);

EXPORT void* orc_model_create(const orc_config* cfg, uint64_t seed, float wscale) {
  orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
  m->c = *cfg; m->seed = seed; m->scale = wscale;
  const orc_config* c = &m->c;
  if (c->arch == 1) return mla_model_create(m);
  const int NQKV = (c->NH + 2 * c->NKV) * c->HD;
  m->embed = gen_tensor(seed, sid(S_EMBED, -1, 0), (size_t)c->V * c->H, wscale);
  m->lm_head = gen_tensor(seed, sid(S_LMHEAD, -1, 0), (size_t)c->V * c->H, wscale);
  m->batch = c->batch > 1 ? c->batch : 1;
  /* the library's rule for its matrix-core tiles (etxmk_config: batch capacity >= 8, MoE, whole blocks) */
  {
    const int tb = c->wdtype == 1 ? 1024 : 512;
    m->mfma = c->batch >= 8 && c->moe && c->wdtype != 2 && c->H % tb == 0 && c->H / tb <= 8 &&
              (c->NH * c->HD) % tb == 0 && (c->NH * c->HD) / tb <= 8 && c->H / 512 <= 8 && c->E % 16 == 0 &&
              c->MI % 256 == 0 && c->MI <= 4096 && c->V % 16 == 0;
  }
  m->nbps = (c->max_ctx + c->block_size - 1) / c->block_size;
  m->nblocks = m->batch * m->nbps;               /* one paged pool shared by the sequences of the batch */
  m->btab = (int32_t*)malloc(sizeof(int32_t) * (size_t)m->nblocks);
  for (int i = 0; i < m->nblocks; ++i) m->btab[i] = i;
  m->ly = (orc_layer*)calloc((size_t)c->L, sizeof(orc_layer));
  const size_t kvn = (size_t)m->nblocks * c->block_size * c->NKV * c->HD;
  for (int l = 0; l < c->L; ++l) {
    orc_layer* y = &m->ly[l];
    y->wqkv = gen_mat(seed, sid(S_WQKV, l, 0), (size_t)NQKV, c->H, wscale, c->wdtype);
    y->wo = gen_mat(seed, sid(S_WO, l, 0), (size_t)c->H, c->NH * c->HD, wscale, c->wdtype);
    if (c->moe) {
      y->wr = gen_tensor(seed, sid(S_ROUTER, l, 0), (size_t)c->E * c->H, wscale);
      y->w13 = (orc_mat*)calloc((size_t)c->E, sizeof(orc_mat));
      y->w2 = (orc_mat*)calloc((size_t)c->E, sizeof(orc_mat));
    } else {
      y->wgu = gen_mat(seed, sid(S_WGU, l, 0), (size_t)2 * c->I, c->H, wscale, c->wdtype);
      y->wd = gen_mat(seed, sid(S_WD, l, 0), (size_t)c->H, c->I, wscale, c->wdtype);
    }
    y->kc = (uint16_t*)calloc(kvn, sizeof(uint16_t));
    y->vc = (uint16_t*)calloc(kvn, sizeof(uint16_t));
  }
  const int half = c->HD / 2;
  m->rcos = (float*)malloc(sizeof(float) * (size_t)c->max_ctx * half);
  m->rsin = (float*)malloc(sizeof(float) * (size_t)c->max_ctx * half);
  orc_rope_tables(c->theta, c->HD, c->max_ctx, m->rcos, m->rsin);
  return m;
}

EXPORT void orc_model_destroy(void* h) {
  orc_model* m = (orc_model*)h;
  if (!m) return;
  for (int l = 0; l < m->c.L; ++l) {
    orc_layer* y = &m->ly[l];
    free_mat(&y->wqkv); free_mat(&y->wo); free(y->wr); free_mat(&y->wgu); free_mat(&y->wd); free(y->kc); free(y->vc);
    free(y->wkvb); free_mat(&y->wsgu); free_mat(&y->wsd);
    if (y->w13) for (int e = 0; e < m->c.E; ++e) { free_mat(&y->w13[e]); free_mat(&y->w2[e]); }
    free(y->w13); free(y->w2);
  }
  free(m->ly); free(m->embed); free(m->lm_head); free(m->btab); free(m->rcos); free(m->rsin); free(m);
}

/* block table override, [batch][blocks per sequence] flattened: entry b * nbps + i is the physical block of
 * sequence b's logical block i (examples/vllm_llm/host.hip:279-282 uploads the same table) */
EXPORT void orc_set_block_table(void* h, const int32_t* bt, int n) {
  orc_model* m = (orc_model*)h;
  for (int i = 0; i < n && i < m->nblocks; ++i) m->btab[i] = bt[i];
}
EXPORT int orc_num_blocks(void* h) { return ((orc_model*)h)->nblocks; }
EXPORT int orc_blocks_per_seq(void* h) { return ((orc_model*)h)->nbps; }
EXPORT const uint16_t* orc_kcache(void* h, int layer) { return ((orc_model*)h)->ly[layer].kc; }
EXPORT const uint16_t* orc_vcache(void* h, int layer) { return ((orc_model*)h)->ly[layer].vc; }

/* fill positions [0, n) of sequence `seq`'s cache in every layer with bf16 N(0,1) (the single-layer
 * configuration; the batched workloads' contexts): element (t, h, d) is number (t*NKV + h)*HD + d of the
 * layer's K / V stream for that sequence */
EXPORT void orc_fill_latent_random_seq(void* h, int seq, int n);
EXPORT void orc_fill_kv_random_seq(void* h, int seq, int n) {
  orc_model* m = (orc_model*)h; const orc_config* c = &m->c;
  if (c->arch == 1) { orc_fill_latent_random_seq(h, seq, n); return; }
  const int NKV = c->NKV, HD = c->HD, BS = c->block_size;
  const int32_t* bt = m->btab + (size_t)seq * m->nbps;
  for (int l = 0; l < c->L; ++l) {
    const uint64_t kk = stream_key(m->seed, sid(S_KINIT, l, seq)), vk = stream_key(m->seed, sid(S_VINIT, l, seq));
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n; ++t)
      for (int hh = 0; hh < NKV; ++hh)
        for (int d = 0; d < HD; ++d) {
          const uint64_t idx = ((uint64_t)t * NKV + hh) * HD + d;
          const int blk = bt[t / BS], off = t % BS;
          m->ly[l].kc[kv_k_index(blk, off, hh, d, NKV, HD, BS)] = f2bf(mk_normal(kk, idx));
          m->ly[l].vc[kv_v_index(blk, off, hh, d, NKV, HD, BS)] = f2bf(mk_normal(vk, idx));
        }
  }
}
EXPORT void orc_fill_kv_random(void* h, int n) { orc_fill_kv_random_seq(h, 0, n); }

static int mla_cache_dim(const orc_config* c) { return c->kv_lora + c->qk_rope; }

static void ensure_expert(orc_model* m, int l, int e) {
  const orc_config* c = &m->c;
  orc_layer* y = &m->ly[l];
  if (!y->w13[e].w && !y->w13[e].q) y->w13[e] = gen_mat(m->seed, sid(S_W13, l, e), (size_t)2 * c->MI, c->H, m->scale, c->wdtype);
  if (!y->w2[e].w && !y->w2[e].q) y->w2[e] = gen_mat(m->seed, sid(S_W2, l, e), (size_t)c->H, c->MI, m->scale, c->wdtype);
}

/* GEMV rows [0, R) of a weight matrix into out, rounding each to bf16 */
static void gemv_mat(const orc_mat* W, int wdtype, int R, int K, const float* x, float* out) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < R; ++r) out[r] = bfr(mat_dot(W, wdtype, (size_t)r, x, K));
}
/* GEMV rows [0, R) into out, rounding each to bf16 */
static void gemv_bf(const uint16_t* W, int R, int K, const float* x, float* out) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < R; ++r) out[r] = bfr(dot64(W + (size_t)r * K, x, K));
}

/* one decoder layer at position pos on residual x (in place) of the sequence whose block table is bt;
 * dump_ids / dump_wts / dump_logits optional */
static float gateup_dot(const orc_model* m, const orc_mat* W, int wdtype, size_t r, const float* x, int K);
static void down_rows(const orc_model* m, const orc_mat* W2, int wdtype, int H, int MI, const float* h, float w,
                      float* out);
static void gemv_rows_tiles(const orc_mat* W, int wdtype, int R, int K, const float* X, int ldx, int n, float* out,
                            int ldo);
/* a dense projection of one vector: the matrix-core tile order for models whose batched kernel uses it */
static void proj_mat(const orc_model* m, const orc_mat* W, int wdtype, int R, int K, const float* x, float* out) {
  if (m->mfma) gemv_rows_tiles(W, wdtype, R, K, x, K, 1, out, R);
  else gemv_mat(W, wdtype, R, K, x, out);
}
static void layer_step(orc_model* m, int l, float* x, int pos, const int32_t* bt, int32_t* ids_out, float* wts_out,
                       float* logits_out) {
  const orc_config* c = &m->c;
  orc_layer* y = &m->ly[l];
  const int H = c->H, NH = c->NH, NKV = c->NKV, HD = c->HD, G = NH / NKV, BS = c->block_size;
  const int NQKV = (NH + 2 * NKV) * HD;
  float* xs = (float*)malloc(sizeof(float) * (size_t)(H > c->I ? H : c->I) * 2 + 64);
  float* qkv = (float*)malloc(sizeof(float) * (size_t)NQKV);
  float* o = (float*)malloc(sizeof(float) * (size_t)NH * HD);
  rmsnorm(x, NULL, H, c->eps, xs);                                 /* input_layernorm (weight 1.0) */
  const int wt = c->wdtype;
  proj_mat(m, &y->wqkv, wt, NQKV, H, xs, qkv);                     /* :112-115 */
  const float* cs = m->rcos + (size_t)pos * (HD / 2);
  const float* sn = m->rsin + (size_t)pos * (HD / 2);
  float tmp[512];
  for (int hh = 0; hh < NH + NKV; ++hh) {                          /* :116-120 q/k norm, RoPE */
    float* v = qkv + (size_t)hh * HD;
    if (c->qk_norm) { rmsnorm(v, NULL, HD, c->eps, tmp); memcpy(v, tmp, sizeof(float) * (size_t)HD); }
    apply_rope(v, HD, cs, sn);
  }
  const int blk = bt[pos / BS], off = pos % BS;                    /* :121 KV append, paged */
  for (int hh = 0; hh < NKV; ++hh)
    for (int d = 0; d < HD; ++d) {
      y->kc[kv_k_index(blk, off, hh, d, NKV, HD, BS)] = f2bf(qkv[(size_t)(NH + hh) * HD + d]);
      y->vc[kv_v_index(blk, off, hh, d, NKV, HD, BS)] = f2bf(qkv[(size_t)(NH + NKV + hh) * HD + d]);
    }
#pragma omp parallel for schedule(static)
  for (int hh = 0; hh < NH; ++hh)                                   /* :122-129 */
    attention_head(qkv + (size_t)hh * HD, y->kc, y->vc, bt, pos + 1, hh / G, NKV, HD, BS, o + (size_t)hh * HD);
  float* t = (float*)malloc(sizeof(float) * (size_t)(H > c->I ? H : c->I) * 2 + 64);
  proj_mat(m, &y->wo, wt, H, NH * HD, o, t);                       /* :130 */
  for (int i = 0; i < H; ++i) x[i] = bfr(x[i] + t[i]);
  rmsnorm(x, NULL, H, c->eps, xs);                                 /* :131 post_attention_layernorm */
  if (c->moe) {
    const int E = c->E, K = c->TOPK, MI = c->MI;
    float logits[1024];
    if (m->mfma) {                                                   /* :134 */
      const orc_mat wr = {y->wr, NULL, NULL};
      gemv_rows_tiles(&wr, 0, E, H, xs, H, 1, logits, E);
    } else {
      gemv_bf(y->wr, E, H, xs, logits);
    }
    if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t)E);
    int32_t ids[64]; float wts[64];
    route(logits, E, K, c->norm_topk, ids, wts);                     /* :135-140 */
    if (ids_out) memcpy(ids_out, ids, sizeof(int32_t) * (size_t)K);
    if (wts_out) memcpy(wts_out, wts, sizeof(float) * (size_t)K);
    for (int k = 0; k < K; ++k) ensure_expert(m, l, ids[k]);
    int order[64];                                                   /* :141 ascending expert id */
    for (int k = 0; k < K; ++k) order[k] = k;
    for (int a = 1; a < K; ++a)
      for (int b = a; b > 0 && ids[order[b]] < ids[order[b - 1]]; --b) { int q = order[b]; order[b] = order[b - 1]; order[b - 1] = q; }
    float* hbuf = (float*)malloc(sizeof(float) * (size_t)K * MI);
    float* ys = (float*)malloc(sizeof(float) * (size_t)K * H);
    for (int k = 0; k < K; ++k) {                                    /* :142-146 */
      const orc_mat* W13 = &y->w13[ids[k]];
      float* hk = hbuf + (size_t)k * MI;
#pragma omp parallel for schedule(static)
      for (int j = 0; j < MI; ++j) {
        const float g = bfr(gateup_dot(m, W13, wt, (size_t)(2 * j), xs, H));
        const float u = bfr(gateup_dot(m, W13, wt, (size_t)(2 * j + 1), xs, H));
        hk[j] = bfr(bfr(silu(g)) * u);
      }
      down_rows(m, &y->w2[ids[k]], wt, H, MI, hk, wts[k], ys + (size_t)k * H);
    }
    for (int i = 0; i < H; ++i) {                                    /* :146-148 */
      float acc = 0.0f;
      for (int k = 0; k < K; ++k) acc = bfr(acc + ys[(size_t)order[k] * H + i]);
      x[i] = bfr(x[i] + acc);
    }
    free(hbuf); free(ys);
  } else {                                                           /* :149-152 */
    const int I = c->I;
    float* hb = (float*)malloc(sizeof(float) * (size_t)I);
#pragma omp parallel for schedule(static)
    for (int j = 0; j < I; ++j) {
      const float g = bfr(mat_dot(&y->wgu, wt, (size_t)(2 * j), xs, H));
      const float u = bfr(mat_dot(&y->wgu, wt, (size_t)(2 * j + 1), xs, H));
      hb[j] = bfr(bfr(silu(g)) * u);
    }
    gemv_mat(&y->wd, wt, H, I, hb, t);
    for (int i = 0; i < H; ++i) x[i] = bfr(x[i] + t[i]);
    free(hb);
  }
  free(xs); free(qkv); free(o); free(t);
}

/* ------------------------------------------------------------------ many rows at once */
/* A row is one decode step of one sequence: its token, position and block table.  orc_step_rows computes n rows
 * with the loops turned round: every weight row is read once and dotted with the n rows' vectors, each in the
 * canonical order of dot64; each layer writes the K/V of every row before any row attends, and row r attends to
 * its own sequence's positions up to its own.  So n rows of distinct sequences are one batched step (each row what
 * orc_step_seq computes), and n consecutive positions of one sequence are the prompt loop of
 * examples/llm/host.hip:203-213 (each position what the decode step at that position computes, given the earlier
 * positions' K/V).  tests/test_oracle_prefill.py checks both forms against orc_step_seq bit for bit. */
typedef struct {
  const int32_t* bt;   /* the row's sequence's block table */
  int pos;             /* the row's position */
} orc_row;

/* row r of a matrix as fp32 weights, with the factor its dot is multiplied by (the fp8 row scale, else 1) */
static inline float row_f32(const orc_mat* m, int wdtype, size_t r, int K, float* out) {
  if (wdtype == 0) { for (int k = 0; k < K; ++k) out[k] = bf2f(m->w[r * K + k]); return 1.0f; }
  if (wdtype == 1) { for (int k = 0; k < K; ++k) out[k] = e4m3_f(m->q[r * K + k]); return m->s[r]; }
  for (int k = 0; k < K; ++k) out[k] = bfr(e4m3_f(m->q[r * K + k]) * m->s[r]);
  return 1.0f;
}
/* dot64 with fp32 weights: the same fma chain per lane and the same lane reduction, in AVX2.  Lane l of the 64 is
 * element l of ymm accumulator l / 8.  lanes_reduce() adds partners l^1, l^2, then the 8-lane and 16-lane mirrors and
 * the rows pairwise: for the sum it returns (every step is one addition of two values, and a + b == b + a) that is
 * the balanced pairwise tree over lanes 0..63 in order, ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7)) per eight,
 * eights paired, then (R0 + R1) + (R2 + R3).  Two hadd rounds build the tree of each eight in a 128-bit half,
 * adding the halves closes it.  tests/test_oracle_prefill.py compares this with dot64 on random rows. */
static inline float tree64(const __m256 v[8]) {
  const __m256 h01 = _mm256_hadd_ps(v[0], v[1]), h23 = _mm256_hadd_ps(v[2], v[3]);
  const __m256 h45 = _mm256_hadd_ps(v[4], v[5]), h67 = _mm256_hadd_ps(v[6], v[7]);
  const __m256 k0 = _mm256_hadd_ps(h01, h23), k1 = _mm256_hadd_ps(h45, h67);   /* [G0 G1 G2 G3 | G0' ...] halves */
  const __m128 g03 = _mm_add_ps(_mm256_castps256_ps128(k0), _mm256_extractf128_ps(k0, 1));   /* G0..G3 */
  const __m128 g47 = _mm_add_ps(_mm256_castps256_ps128(k1), _mm256_extractf128_ps(k1, 1));   /* G4..G7 */
  float g[8];
  _mm_storeu_ps(g, g03);
  _mm_storeu_ps(g + 4, g47);
  return ((g[0] + g[1]) + (g[2] + g[3])) + ((g[4] + g[5]) + (g[6] + g[7]));
}
static inline float dot64f(const float* w, const float* x, int K) {
  __m256 a[8];
  for (int j = 0; j < 8; ++j) a[j] = _mm256_setzero_ps();
  for (int k0 = 0; k0 < K; k0 += 64)
    for (int j = 0; j < 8; ++j)
      a[j] = _mm256_fmadd_ps(_mm256_loadu_ps(w + k0 + 8 * j), _mm256_loadu_ps(x + k0 + 8 * j), a[j]);
  return tree64(a);
}
EXPORT float orc_dot64f(const float* w, const float* x, int K) { return dot64f(w, x, K); }

/* ------------------------------------------------------------------ the gfx950 bf16 matrix-core step */
/* One output element of v_mfma_f32_16x16x32_bf16 (D = C + A B over K = 32), as measured on gfx950: exact
 * integer arithmetic, no floating-point order.  a[32] and b[32] are the bf16 operands in register order (lane quad
 * q holds elements 8q .. 8q+7 of its A row and B column).  The four quads' groups of 8 products enter the fp32
 * accumulator one after another, in quad order:
 *   - a group's products (exact, bf16 x bf16) are aligned to E, the largest sum of the two operands' exponents in
 *     the group, and each is truncated toward zero to a multiple of 2^(E-24); the group sum S is their exact sum;
 *   - the accumulator is floored to a multiple of 2^(E-24); when the accumulator's exponent Ea exceeds E + 7, S is
 *     floored to a multiple of 2^(Ea-31) instead (8 bits below the accumulator's last bit);
 *   - the exact sum of the two is rounded to fp32, to nearest, ties to even (+0 for an exact zero).
 * A group whose products are all zero leaves the accumulator unchanged.  Operands and results are taken to be
 * normal numbers or zero (bf16 subnormal operands, fp32 overflow and subnormal results are outside this
 * statement).  The statement is pinned by tests/test_oracle_mfma.py against the hardware's outputs on wide-range,
 * cancelling and chained inputs kept in tests/golden/, and by tests/test_gpu_mfma.py against the hardware itself. */
static inline int bf_decomp(uint16_t h, int* e, int* m) {    /* value = s * m * 2^(e - 7); returns the sign */
  const int ex = (h >> 7) & 0xFF;
  *m = ex ? ((h & 0x7F) | 0x80) : (h & 0x7F);
  *e = ex ? ex - 127 : -126;
  return (h & 0x8000) ? -1 : 1;
}
static float rne_scaled(int64_t t, int u) {                  /* fp32 nearest to t * 2^u, ties to even */
  if (t == 0) return 0.0f;
  const int neg = t < 0;
  uint64_t m = neg ? (uint64_t)(-t) : (uint64_t)t;
  int nb = 64 - __builtin_clzll(m);
  if (nb > 24) {
    const int sh = nb - 24;
    uint64_t q = m >> sh, rem = m & ((1ull << sh) - 1), half = 1ull << (sh - 1);
    if (rem > half || (rem == half && (q & 1))) ++q;
    m = q;
    u += sh;
  }
  {                                 /* m <= 2^24 now: a normal result is m * 2^u exactly, built from its bits */
    const int mb = 64 - __builtin_clzll(m);
    uint64_t mm = m;
    int uu = u;
    if (mb < 24) { mm <<= 24 - mb; uu -= 24 - mb; }
    else if (mb == 25) { mm >>= 1; uu += 1; }               /* the carry of a round-up: m == 2^24 */
    const int e = uu + 23;
    if (e >= -126 && e <= 127) {
      const uint32_t bits = (neg ? 0x80000000u : 0u) | ((uint32_t)(e + 127) << 23) | (uint32_t)(mm & 0x7FFFFF);
      float r;
      memcpy(&r, &bits, 4);
      return r;
    }
  }
  const float r = ldexpf((float)m, u);
  return neg ? -r : r;
}
static float mfma_bf16_k32(float acc, const uint16_t* a, const uint16_t* b) {
  for (int q = 0; q < 4; ++q) {
    int sg[8], ep[8];
    int64_t mp[8];
    int E = INT32_MIN;
    for (int j = 0; j < 8; ++j) {
      int ea, ma, eb, mb;
      const int s = bf_decomp(a[8 * q + j], &ea, &ma) * bf_decomp(b[8 * q + j], &eb, &mb);
      sg[j] = s;
      mp[j] = (int64_t)ma * mb;
      ep[j] = ea + eb;
      if (mp[j] && ep[j] > E) E = ep[j];
    }
    if (E == INT32_MIN) continue;
    int64_t S = 0;                                          /* units of 2^(E - 24) */
    for (int j = 0; j < 8; ++j) {
      if (!mp[j]) continue;
      const int sh = E - ep[j];                              /* product / 2^(E-24) = mp << 10 >> sh */
      const int64_t v = sh >= 40 ? 0 : ((mp[j] << 10) >> sh);
      S += sg[j] * v;
    }
    int64_t A = 0;
    int u = E - 24;
    if (acc != 0.0f) {
      uint32_t bits; memcpy(&bits, &acc, 4);
      const int aex = (bits >> 23) & 0xFF;
      const int64_t am = aex ? ((bits & 0x7FFFFF) | 0x800000) : (bits & 0x7FFFFF);
      const int ae = aex ? aex - 127 : -126;                 /* acc = +-am * 2^(ae - 23) */
      const int Ea = ae - 23 + (63 - __builtin_clzll((uint64_t)am));
      const int64_t sa = (bits >> 31) ? -am : am;
      if (Ea > E + 7) {                                      /* the group lies below the accumulator's window */
        u = Ea - 31;
        const int sh = u - (E - 24);                         /* >= 1 */
        S = sh >= 62 ? (S < 0 ? -1 : 0) : (S >> sh);         /* floor (arithmetic shift) */
        A = sa * ((int64_t)1 << (ae - 23 - u));
      } else {
        const int d = ae - 23 - u;                           /* floor of acc on the group's grid */
        A = d >= 0 ? sa * ((int64_t)1 << d) : (d <= -62 ? (sa < 0 ? -1 : 0) : (sa >> -d));
      }
    }
    acc = rne_scaled(A + S, u);
  }
  return acc;
}
EXPORT float orc_mfma_bf16_k32(float acc, const uint16_t* a, const uint16_t* b) { return mfma_bf16_k32(acc, a, b); }
/* n chained steps: acc = step(acc, a + 32 i, b + 32 i) for i = 0 .. n-1 */
EXPORT float orc_mfma_bf16_chain(float acc, const uint16_t* a, const uint16_t* b, int n) {
  for (int i = 0; i < n; ++i) acc = mfma_bf16_k32(acc, a + 32 * i, b + 32 * i);
  return acc;
}

/* The same step on pre-decomposed operands (signed significand with its hidden bit, exponent; zero: significand 0),
 * for the dots the oracle runs many times: identical results to mfma_bf16_k32 (tests/test_oracle_mfma.py). */
static inline void bf_split(uint16_t h, int16_t* m, int16_t* e) {
  int ee, mm;
  const int sg = bf_decomp(h, &ee, &mm);
  *m = (int16_t)(sg * mm);
  *e = (int16_t)ee;
}
/* The group's sum S of products truncated toward zero to 2^(E-24), in units of 2^(E-34), and E, with AVX2: the 8
 * products (significand products below 2^16, shifted up by 10 in 64-bit lanes, so a shift of 26 or more leaves 0, as
 * the scalar statement's cut at 40 does); zero products take no part in E and add 0. */
static inline int mfma_group_split(const int16_t* am, const int16_t* ae, const int16_t* bm, const int16_t* be,
                                   int64_t* S) {
  const __m256i a_m = _mm256_cvtepi16_epi32(_mm_loadu_si128((const __m128i*)am));
  const __m256i b_m = _mm256_cvtepi16_epi32(_mm_loadu_si128((const __m128i*)bm));
  const __m256i ep = _mm256_add_epi32(_mm256_cvtepi16_epi32(_mm_loadu_si128((const __m128i*)ae)),
                                      _mm256_cvtepi16_epi32(_mm_loadu_si128((const __m128i*)be)));
  const __m256i mp = _mm256_mullo_epi32(a_m, b_m);
  const __m256i zero = _mm256_setzero_si256();
  const __m256i isz = _mm256_cmpeq_epi32(mp, zero);
  const __m256i epm = _mm256_blendv_epi8(ep, _mm256_set1_epi32(INT32_MIN), isz);
  __m256i mx = _mm256_max_epi32(epm, _mm256_permute2x128_si256(epm, epm, 1));
  mx = _mm256_max_epi32(mx, _mm256_shuffle_epi32(mx, _MM_SHUFFLE(1, 0, 3, 2)));
  mx = _mm256_max_epi32(mx, _mm256_shuffle_epi32(mx, _MM_SHUFFLE(2, 3, 0, 1)));
  const int E = _mm_cvtsi128_si32(_mm256_castsi256_si128(mx));
  if (E == INT32_MIN) return E;
  const __m256i sh = _mm256_sub_epi32(_mm256_set1_epi32(E), ep);   /* >= 0 for every non-zero product */
  const __m256i mag = _mm256_abs_epi32(mp);
  const __m256i neg = _mm256_cmpgt_epi32(zero, mp);
  __m256i v_lo = _mm256_slli_epi64(_mm256_cvtepu32_epi64(_mm256_castsi256_si128(mag)), 10);
  __m256i v_hi = _mm256_slli_epi64(_mm256_cvtepu32_epi64(_mm256_extracti128_si256(mag, 1)), 10);
  v_lo = _mm256_srlv_epi64(v_lo, _mm256_cvtepu32_epi64(_mm256_castsi256_si128(sh)));
  v_hi = _mm256_srlv_epi64(v_hi, _mm256_cvtepu32_epi64(_mm256_extracti128_si256(sh, 1)));
  const __m256i n_lo = _mm256_cvtepi32_epi64(_mm256_castsi256_si128(neg));
  const __m256i n_hi = _mm256_cvtepi32_epi64(_mm256_extracti128_si256(neg, 1));
  v_lo = _mm256_sub_epi64(_mm256_xor_si256(v_lo, n_lo), n_lo);
  v_hi = _mm256_sub_epi64(_mm256_xor_si256(v_hi, n_hi), n_hi);
  const __m256i s4 = _mm256_add_epi64(v_lo, v_hi);
  const __m128i s2 = _mm_add_epi64(_mm256_castsi256_si128(s4), _mm256_extracti128_si256(s4, 1));
  *S = _mm_cvtsi128_si64(s2) + _mm_extract_epi64(s2, 1);
  return E;
}
static float mfma_step_split(float acc, const int16_t* am, const int16_t* ae, const int16_t* bm, const int16_t* be) {
  for (int q = 0; q < 4; ++q) {
    int64_t S;
    const int E = mfma_group_split(am + 8 * q, ae + 8 * q, bm + 8 * q, be + 8 * q, &S);
    if (E == INT32_MIN) continue;
    int64_t A = 0;
    int u = E - 24;
    if (acc != 0.0f) {
      uint32_t bits; memcpy(&bits, &acc, 4);
      const int aex = (bits >> 23) & 0xFF;
      const int64_t am2 = aex ? ((bits & 0x7FFFFF) | 0x800000) : (bits & 0x7FFFFF);
      const int ae2 = aex ? aex - 127 : -126;
      const int Ea = ae2 - 23 + (63 - __builtin_clzll((uint64_t)am2));
      const int64_t sa = (bits >> 31) ? -am2 : am2;
      if (Ea > E + 7) {
        u = Ea - 31;
        const int sh = u - (E - 24);
        S = sh >= 62 ? (S < 0 ? -1 : 0) : (S >> sh);
        A = sa * ((int64_t)1 << (ae2 - 23 - u));
      } else {
        const int d = ae2 - 23 - u;
        A = d >= 0 ? sa * ((int64_t)1 << d) : (d <= -62 ? (sa < 0 ? -1 : 0) : (sa >> -d));
      }
    }
    acc = rne_scaled(A + S, u);
  }
  return acc;
}
/* The order of the batched kernels' matrix-core gate/up tiles over a row of K (a multiple of 512): 512-element
 * blocks ascending; in a block 16 steps, step s giving lane quad q the 8 elements 4s + q + 64 j, j = 0 .. 7 (the
 * 16-byte lane slot 4s + q of the lane-permuted layout; for e4m3 rows the two halves of a 1024-block's slot are the
 * same slot of two consecutive 512-blocks).  mfma_split_row permutes and decomposes a row of fp32 values holding bf16
 * (or e4m3) values into that order, mfma_dot_split runs the chain from 0. */
static void mfma_split_row(const float* v, int K, int16_t* m, int16_t* e) {
  for (int blk = 0; blk < K / 512; ++blk)
    for (int s = 0; s < 16; ++s)
      for (int q = 0; q < 4; ++q)
        for (int j = 0; j < 8; ++j) {
          const size_t o = (size_t)blk * 512 + 32 * s + 8 * q + j;
          bf_split(f2bf(v[512 * blk + 4 * s + q + 64 * j]), m + o, e + o);
        }
}
static float mfma_dot_split(const int16_t* am, const int16_t* ae, const int16_t* bm, const int16_t* be, int K) {
  float acc = 0.0f;
  for (int st = 0; st < K / 32; ++st)
    acc = mfma_step_split(acc, am + 32 * st, ae + 32 * st, bm + 32 * st, be + 32 * st);
  return acc;
}
/* x[K] (fp32 values holding bf16) . w[K] (fp32 values holding bf16 or e4m3) in the tile order */
/* an expert gate/up row's value before its bf16 rounding: the matrix-core tile order for models whose batched kernel
 * uses it (m->mfma), else mat_dot */
static float gateup_dot(const orc_model* m, const orc_mat* W, int wdtype, size_t r, const float* x, int K) {
  if (!m->mfma) return mat_dot(W, wdtype, r, x, K);
  float* wf = (float*)malloc(sizeof(float) * (size_t)K);
  int16_t* buf = (int16_t*)malloc(sizeof(int16_t) * 4 * (size_t)K);
  const float sc = row_f32(W, wdtype, r, K, wf);
  mfma_split_row(wf, K, buf, buf + K);
  mfma_split_row(x, K, buf + 2 * K, buf + 3 * K);
  const float d = mfma_dot_split(buf, buf + K, buf + 2 * K, buf + 3 * K, K) * sc;
  free(wf); free(buf);
  return d;
}
EXPORT float orc_mfma_tile_dot(const float* w, const float* x, int K) {
  int16_t* buf = (int16_t*)malloc(sizeof(int16_t) * 4 * (size_t)K);
  mfma_split_row(w, K, buf, buf + K);
  mfma_split_row(x, K, buf + 2 * K, buf + 3 * K);
  const float r = mfma_dot_split(buf, buf + K, buf + 2 * K, buf + 3 * K, K);
  free(buf);
  return r;
}
/* logical element k of a stored row of K -> its stored position: blocks of blk (512 for bf16 rows, 1024 for e4m3
 * rows; a last block of 64m gives each lane m), lane l of a block holding l, l + 64, ... (the library's
 * perm_stored / perm_stored8) */
static int stored_pos(int k, int K, int blk) {
  const int base = k & ~(blk - 1), S = K - base < blk ? K - base : blk, m = S >> 6, q = k - base;
  return base + (q & 63) * m + (q >> 6);
}
/* The order of the batched kernels' matrix-core expert down tiles over a row of K (a multiple of 256): the down row's
 * stored positions ascending, step s giving lane quad q positions 32s + 8q .. + 7 (the pairs' h rows are stored in
 * the same order).  mfma_split_stored decomposes a row of fp32 values holding bf16 (or e4m3) values into it. */
static void mfma_split_stored(const float* v, int K, int blk, int16_t* m, int16_t* e) {
  for (int k = 0; k < K; ++k) {
    const int o = stored_pos(k, K, blk);
    bf_split(f2bf(v[k]), m + o, e + o);
  }
}
/* out[i] = bfr(bfr(down row i . h) * w) for rows [0, H): the matrix-core stored order for models whose batched kernel
 * uses it (m->mfma), else mat_dot */
static void down_rows(const orc_model* m, const orc_mat* W2, int wdtype, int H, int MI, const float* h, float w,
                      float* out) {
  if (!m->mfma) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < H; ++i) out[i] = bfr(bfr(mat_dot(W2, wdtype, (size_t)i, h, MI)) * w);
    return;
  }
  const int blk = wdtype == 1 ? 1024 : 512;
  int16_t* hsp = (int16_t*)malloc(sizeof(int16_t) * 2 * (size_t)MI);
  mfma_split_stored(h, MI, blk, hsp, hsp + MI);
#pragma omp parallel
  {
    float* wf = (float*)malloc(sizeof(float) * (size_t)MI);
    int16_t* wsp = (int16_t*)malloc(sizeof(int16_t) * 2 * (size_t)MI);
#pragma omp for schedule(static)
    for (int i = 0; i < H; ++i) {
      const float sc = row_f32(W2, wdtype, (size_t)i, MI, wf);
      mfma_split_stored(wf, MI, blk, wsp, wsp + MI);
      out[i] = bfr(bfr(mfma_dot_split(wsp, wsp + MI, hsp, hsp + MI, MI) * sc) * w);
    }
    free(wf); free(wsp);
  }
  free(hsp);
}
EXPORT float orc_mfma_down_dot(const float* w, const float* h, int K, int blk) {
  if (K % 256 || (blk != 512 && blk != 1024)) return NAN;
  int16_t* buf = (int16_t*)malloc(sizeof(int16_t) * 4 * (size_t)K);
  mfma_split_stored(w, K, blk, buf, buf + K);
  mfma_split_stored(h, K, blk, buf + 2 * K, buf + 3 * K);
  const float r = mfma_dot_split(buf, buf + K, buf + 2 * K, buf + 3 * K, K);
  free(buf);
  return r;
}
/* value of row r for vector x: mat_dot's result, from the row's fp32 image */
static inline float row_dot(const float* wf, float sc, int wdtype, const float* x, int K) {
  const float d = dot64f(wf, x, K);
  return wdtype == 1 ? d * sc : d;
}
/* out[b * ldo + r] = bfr(row r . X[b * ldx ..]) for rows [0, R), vectors [0, n).  A thread takes 8 rows at a time
 * (their fp32 images stay in its L2) and runs every vector against them (each vector stays in L1 for the 8). */
#define ORC_TR 8
static void gemv_rows_multi(const orc_mat* W, int wdtype, int R, int K, const float* X, int ldx, int n, float* out,
                            int ldo) {
#pragma omp parallel
  {
    float* wf = (float*)malloc(sizeof(float) * (size_t)K * ORC_TR);
    float sc[ORC_TR];
#pragma omp for schedule(dynamic, 1)
    for (int r0 = 0; r0 < R; r0 += ORC_TR) {
      const int nr = R - r0 < ORC_TR ? R - r0 : ORC_TR;
      for (int i = 0; i < nr; ++i) sc[i] = row_f32(W, wdtype, (size_t)(r0 + i), K, wf + (size_t)i * K);
      for (int b = 0; b < n; ++b)
        for (int i = 0; i < nr; ++i)
          out[(size_t)b * ldo + r0 + i] = bfr(row_dot(wf + (size_t)i * K, sc[i], wdtype, X + (size_t)b * ldx, K));
    }
    free(wf);
  }
}

/* a dense projection row's value before scaling in the split order (decomposed operands in the tile order, blocks of
 * TBK, a power-of-two count up to 8): each block's chain from zero, then the pairwise tree of the partials */
static float proj_split_dot(const int16_t* am, const int16_t* ae, const int16_t* bm, const int16_t* be, int K, int TBK) {
  const int nb = K / TBK;
  float t[8];
  for (int k = 0; k < nb; ++k) t[k] = mfma_dot_split(am + k * TBK, ae + k * TBK, bm + k * TBK, be + k * TBK, TBK);
  for (int width = 1; width < nb; width *= 2)
    for (int k = 0; k + width < nb; k += 2 * width) t[k] = t[k] + t[k + width];
  return t[0];
}
EXPORT float orc_mfma_proj_dot(const float* w, const float* x, int K, int TBK) {
  if (TBK <= 0 || K % TBK || K / TBK > 8 || ((K / TBK) & (K / TBK - 1))) return NAN;
  int16_t* buf = (int16_t*)malloc(sizeof(int16_t) * 4 * (size_t)K);
  mfma_split_row(w, K, buf, buf + K);
  mfma_split_row(x, K, buf + 2 * K, buf + 3 * K);
  const float r = proj_split_dot(buf, buf + K, buf + 2 * K, buf + 3 * K, K, TBK);
  free(buf);
  return r;
}
/* gemv_rows_multi in the batched kernels' split tile order for the dense projections: the row's blocks (512
 * elements, 1024 for e4m3 rows) each run the tile chain from zero, and the partials are added as a pairwise tree
 * ((P0 + P1) + (P2 + P3)) ... (a block count of 1, 2, 4 or 8), then scaled; each vector decomposed once, each row
 * once per thread */
static void gemv_rows_tiles(const orc_mat* W, int wdtype, int R, int K, const float* X, int ldx, int n, float* out,
                            int ldo) {
  const int TBK = wdtype == 1 ? 1024 : 512;
  int16_t* xsp = (int16_t*)malloc(sizeof(int16_t) * 2 * (size_t)n * K);
  for (int b = 0; b < n; ++b) mfma_split_row(X + (size_t)b * ldx, K, xsp + 2 * (size_t)b * K, xsp + (2 * (size_t)b + 1) * K);
#pragma omp parallel
  {
    float* wf = (float*)malloc(sizeof(float) * (size_t)K);
    int16_t* wsp = (int16_t*)malloc(sizeof(int16_t) * 2 * (size_t)K);
#pragma omp for schedule(dynamic, 8)
    for (int r = 0; r < R; ++r) {
      const float sc = row_f32(W, wdtype, (size_t)r, K, wf);
      mfma_split_row(wf, K, wsp, wsp + K);
      for (int b = 0; b < n; ++b) {
        const int16_t* xm = xsp + 2 * (size_t)b * K;
        out[(size_t)b * ldo + r] = bfr(proj_split_dot(wsp, wsp + K, xm, xm + K, K, TBK) * sc);
      }
    }
    free(wf); free(wsp);
  }
  free(xsp);
}

/* attention_head for every row's q heads (row r's at qkv + r * ldq).  Rows of one sequence share one gathered copy of
 * that sequence's cache, fp32 K^T [h][d][t] and V [h][t][d] over positions 0 .. (largest position of its rows): the
 * scores of eight positions are computed at a time (each one's fma chain over d ascending, as in attention_head),
 * and a[d] for eight dims at a time (each one's chain over t ascending).  The chunk maxima, the exponentials, the
 * chunk sums and the merge are attention_head's, in its order. */
static void attention_rows(const uint16_t* kc, const uint16_t* vc, const orc_row* rows, int n, const float* qkv, int ldq,
                           int NH, int NKV, int HD, int BS, float* o) {
  const int G = NH / NKV;
  const float scale = (float)(1.0 / sqrt((double)HD));
  int* done = (int*)calloc((size_t)n, sizeof(int));
  int* grp = (int*)malloc(sizeof(int) * (size_t)n);
  for (int r0 = 0; r0 < n; ++r0) {
    if (done[r0]) continue;
    const int32_t* bt = rows[r0].bt;
    int ng = 0, T = 0;
    for (int r = r0; r < n; ++r)
      if (!done[r] && rows[r].bt == bt) {
        done[r] = 1;
        grp[ng++] = r;
        if (rows[r].pos + 1 > T) T = rows[r].pos + 1;
      }
    const int Tp = (T + 7) & ~7;
    float* kt = (float*)malloc(sizeof(float) * (size_t)NKV * HD * Tp);
    float* vt = (float*)malloc(sizeof(float) * (size_t)NKV * Tp * HD);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < Tp; ++t)
      for (int h = 0; h < NKV; ++h)
        for (int d = 0; d < HD; ++d) {
          float kv = 0.0f, vv = 0.0f;
          if (t < T) {
            const int blk = bt[t / BS], off = t % BS;
            kv = bf2f(kc[kv_k_index(blk, off, h, d, NKV, HD, BS)]);
            vv = bf2f(vc[kv_v_index(blk, off, h, d, NKV, HD, BS)]);
          }
          kt[((size_t)h * HD + d) * Tp + t] = kv;
          vt[((size_t)h * Tp + t) * HD + d] = vv;
        }
#pragma omp parallel
    {
      float* sc = (float*)malloc(sizeof(float) * (size_t)Tp);
      float A[512], a[512];
#pragma omp for schedule(dynamic, 1)
      for (int gh = 0; gh < ng * NH; ++gh) {
        const int r = grp[gh / NH], hh = gh % NH, h = hh / G, nt = rows[r].pos + 1, ntp = (nt + 7) & ~7;
        const float* q = qkv + (size_t)r * ldq + (size_t)hh * HD;
        const float* K = kt + (size_t)h * HD * Tp;
        const float* Vv = vt + (size_t)h * Tp * HD;
        for (int t = 0; t < ntp; ++t) sc[t] = 0.0f;
        for (int d = 0; d < HD; ++d) {
          const float qd = q[d];
          const float* kr = K + (size_t)d * Tp;
          for (int t = 0; t < ntp; ++t) sc[t] = fmaf(qd, kr[t], sc[t]);
        }
        for (int t = 0; t < nt; ++t) sc[t] = sc[t] * scale;
        const int nch = (nt + ATT_CHUNK - 1) / ATT_CHUNK;
        float mc[256], M = -INFINITY, L = 0.0f;
        for (int c = 0; c < nch; ++c) {
          const int t0 = c * ATT_CHUNK, t1 = t0 + ATT_CHUNK < nt ? t0 + ATT_CHUNK : nt;
          float m = -INFINITY;
          for (int t = t0; t < t1; ++t) if (sc[t] > m) m = sc[t];
          mc[c] = m;
          if (m > M) M = m;
        }
        for (int d = 0; d < HD; ++d) A[d] = 0.0f;
        for (int c = 0; c < nch; ++c) {
          const int t0 = c * ATT_CHUNK, t1 = t0 + ATT_CHUNK < nt ? t0 + ATT_CHUNK : nt;
          float l = 0.0f;
          for (int d = 0; d < HD; ++d) a[d] = 0.0f;
          for (int t = t0; t < t1; ++t) {
            const float p = mk_expf(sc[t] - mc[c]);
            l = l + p;
            const float* vr = Vv + (size_t)t * HD;
            for (int d = 0; d < HD; ++d) a[d] = fmaf(p, vr[d], a[d]);
          }
          const float w = mk_expf(mc[c] - M);
          L = fmaf(w, l, L);
          for (int d = 0; d < HD; ++d) A[d] = fmaf(w, a[d], A[d]);
        }
        float* ob = o + (size_t)r * NH * HD + (size_t)hh * HD;
        for (int d = 0; d < HD; ++d) ob[d] = bfr(A[d] / L);
      }
      free(sc);
    }
    free(kt);
    free(vt);
  }
  free(done);
  free(grp);
}

/* layer l for n rows; X [n][H] residuals in place; ids_out / wts_out [n] rows of ldk (may be NULL) */
static void layer_rows(orc_model* m, int l, float* X, int n, const orc_row* rows, int32_t* ids_out, float* wts_out,
                       int ldk) {
  const orc_config* c = &m->c;
  orc_layer* y = &m->ly[l];
  const int H = c->H, NH = c->NH, NKV = c->NKV, HD = c->HD, BS = c->block_size, wt = c->wdtype;
  const int NQKV = (NH + 2 * NKV) * HD;
  float* xs = (float*)malloc(sizeof(float) * (size_t)n * H);
  float* qkv = (float*)malloc(sizeof(float) * (size_t)n * NQKV);
  float* o = (float*)malloc(sizeof(float) * (size_t)n * NH * HD);
  float* t = (float*)malloc(sizeof(float) * (size_t)n * H);
  for (int b = 0; b < n; ++b) rmsnorm(X + (size_t)b * H, NULL, H, c->eps, xs + (size_t)b * H);
  if (m->mfma) gemv_rows_tiles(&y->wqkv, wt, NQKV, H, xs, H, n, qkv, NQKV);   /* :112-115 */
  else gemv_rows_multi(&y->wqkv, wt, NQKV, H, xs, H, n, qkv, NQKV);
#pragma omp parallel for schedule(static)
  for (int b = 0; b < n; ++b) {                                                 /* :116-121 */
    float* q = qkv + (size_t)b * NQKV;
    const int pos = rows[b].pos;
    const float* cs = m->rcos + (size_t)pos * (HD / 2);
    const float* sn = m->rsin + (size_t)pos * (HD / 2);
    float tmp[512];
    for (int hh = 0; hh < NH + NKV; ++hh) {
      float* v = q + (size_t)hh * HD;
      if (c->qk_norm) { rmsnorm(v, NULL, HD, c->eps, tmp); memcpy(v, tmp, sizeof(float) * (size_t)HD); }
      apply_rope(v, HD, cs, sn);
    }
    const int blk = rows[b].bt[pos / BS], off = pos % BS;
    for (int hh = 0; hh < NKV; ++hh)
      for (int d = 0; d < HD; ++d) {
        y->kc[kv_k_index(blk, off, hh, d, NKV, HD, BS)] = f2bf(q[(size_t)(NH + hh) * HD + d]);
        y->vc[kv_v_index(blk, off, hh, d, NKV, HD, BS)] = f2bf(q[(size_t)(NH + NKV + hh) * HD + d]);
      }
  }
  attention_rows(y->kc, y->vc, rows, n, qkv, NQKV, NH, NKV, HD, BS, o);         /* :122-129 */
  if (m->mfma) gemv_rows_tiles(&y->wo, wt, H, NH * HD, o, NH * HD, n, t, H);  /* :130 */
  else gemv_rows_multi(&y->wo, wt, H, NH * HD, o, NH * HD, n, t, H);
  for (size_t i = 0; i < (size_t)n * H; ++i) X[i] = bfr(X[i] + t[i]);
  for (int b = 0; b < n; ++b) rmsnorm(X + (size_t)b * H, NULL, H, c->eps, xs + (size_t)b * H);  /* :131 */
  if (c->moe) {
    const int E = c->E, K = c->TOPK, MI = c->MI;
    float* logits = (float*)malloc(sizeof(float) * (size_t)n * E);
    const orc_mat wr = {y->wr, NULL, NULL};
    if (m->mfma) gemv_rows_tiles(&wr, 0, E, H, xs, H, n, logits, E);            /* :134 */
    else gemv_rows_multi(&wr, 0, E, H, xs, H, n, logits, E);
    int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)n * K);
    float* wts = (float*)malloc(sizeof(float) * (size_t)n * K);
    for (int b = 0; b < n; ++b) {
      route(logits + (size_t)b * E, E, K, c->norm_topk, ids + (size_t)b * K, wts + (size_t)b * K);   /* :135-140 */
      if (ids_out) memcpy(ids_out + (size_t)b * ldk, ids + (size_t)b * K, sizeof(int32_t) * (size_t)K);
      if (wts_out) memcpy(wts_out + (size_t)b * ldk, wts + (size_t)b * K, sizeof(float) * (size_t)K);
    }
    /* the (row, slot) pairs grouped by expert: pairs of expert e are pr[pe[e] .. pe[e+1]) */
    int* pe = (int*)calloc((size_t)E + 1, sizeof(int));
    int* pr = (int*)malloc(sizeof(int) * (size_t)n * K);
    for (int i = 0; i < n * K; ++i) pe[ids[i] + 1]++;
    for (int e = 0; e < E; ++e) pe[e + 1] += pe[e];
    int* fill = (int*)malloc(sizeof(int) * (size_t)E);
    memcpy(fill, pe, sizeof(int) * (size_t)E);
    for (int i = 0; i < n * K; ++i) pr[fill[ids[i]]++] = i;
    int* used = (int*)malloc(sizeof(int) * (size_t)E);
    int nu = 0;
    for (int e = 0; e < E; ++e) if (pe[e + 1] > pe[e]) { ensure_expert(m, l, e); used[nu++] = e; }
    float* hb = (float*)malloc(sizeof(float) * (size_t)n * K * MI);           /* h of pair i at hb + i * MI */
    float* ys = (float*)malloc(sizeof(float) * (size_t)n * K * H);            /* y of pair i at ys + i * H */
    int16_t* xsp = NULL;                             /* matrix-core order: the rows' inputs decomposed once */
    if (m->mfma) {
      xsp = (int16_t*)malloc(sizeof(int16_t) * 2 * (size_t)n * H);
#pragma omp parallel for schedule(static)
      for (int i = 0; i < n; ++i) mfma_split_row(xs + (size_t)i * H, H, xsp + 2 * (size_t)i * H, xsp + (2 * (size_t)i + 1) * H);
    }
    int16_t* hsp = m->mfma ? (int16_t*)malloc(sizeof(int16_t) * 2 * (size_t)n * K * MI) : NULL;
#pragma omp parallel
    {
      float* wg = (float*)malloc(sizeof(float) * (size_t)(H > MI ? H : MI) * 2);
      float* wu = wg + (H > MI ? H : MI);
      int16_t* wsp = m->mfma ? (int16_t*)malloc(sizeof(int16_t) * 4 * (size_t)H) : NULL;
#pragma omp for schedule(dynamic, 8)
      for (int u = 0; u < nu * MI; ++u) {                                       /* :142-145 */
        const int e = used[u / MI], j = u % MI;
        const orc_mat* W13 = &y->w13[e];
        const float sg = row_f32(W13, wt, (size_t)(2 * j), H, wg);
        const float su = row_f32(W13, wt, (size_t)(2 * j + 1), H, wu);
        if (wsp) {
          mfma_split_row(wg, H, wsp, wsp + H);
          mfma_split_row(wu, H, wsp + 2 * H, wsp + 3 * H);
        }
        for (int q = pe[e]; q < pe[e + 1]; ++q) {
          const int i = pr[q];
          const float* xb = xs + (size_t)(i / K) * H;
          float g, up;
          if (wsp) {
            const int16_t* xm = xsp + 2 * (size_t)(i / K) * H;
            g = bfr(mfma_dot_split(wsp, wsp + H, xm, xm + H, H) * sg);
            up = bfr(mfma_dot_split(wsp + 2 * H, wsp + 3 * H, xm, xm + H, H) * su);
          } else {
            g = bfr(row_dot(wg, sg, wt, xb, H));
            up = bfr(row_dot(wu, su, wt, xb, H));
          }
          hb[(size_t)i * MI + j] = bfr(bfr(silu(g)) * up);
        }
      }
      free(wsp);
      if (hsp) {                       /* matrix-core order: each pair's h decomposed once, in the down rows' order */
#pragma omp for schedule(static)
        for (int i = 0; i < n * K; ++i)
          mfma_split_stored(hb + (size_t)i * MI, MI, wt == 1 ? 1024 : 512, hsp + 2 * (size_t)i * MI,
                            hsp + (2 * (size_t)i + 1) * MI);
      }
      int16_t* dsp = hsp ? (int16_t*)malloc(sizeof(int16_t) * 2 * (size_t)MI) : NULL;
#pragma omp for schedule(dynamic, 16)
      for (int u = 0; u < nu * H; ++u) {                                        /* :146 */
        const int e = used[u / H], r = u % H;
        const float sd = row_f32(&y->w2[e], wt, (size_t)r, MI, wg);
        if (dsp) mfma_split_stored(wg, MI, wt == 1 ? 1024 : 512, dsp, dsp + MI);
        for (int q = pe[e]; q < pe[e + 1]; ++q) {
          const int i = pr[q];
          const float d = dsp ? mfma_dot_split(dsp, dsp + MI, hsp + 2 * (size_t)i * MI, hsp + (2 * (size_t)i + 1) * MI, MI) * sd
                              : row_dot(wg, sd, wt, hb + (size_t)i * MI, MI);
          ys[(size_t)i * H + r] = bfr(bfr(d) * wts[i]);
        }
      }
      free(dsp);
      free(wg);
    }
    for (int b = 0; b < n; ++b) {                                               /* :146-148 ascending expert id */
      const int32_t* id = ids + (size_t)b * K;
      int order[64];
      for (int k = 0; k < K; ++k) order[k] = k;
      for (int a = 1; a < K; ++a)
        for (int q = a; q > 0 && id[order[q]] < id[order[q - 1]]; --q) { int z = order[q]; order[q] = order[q - 1]; order[q - 1] = z; }
      float* x = X + (size_t)b * H;
      for (int i = 0; i < H; ++i) {
        float acc = 0.0f;
        for (int k = 0; k < K; ++k) acc = bfr(acc + ys[((size_t)b * K + order[k]) * H + i]);
        x[i] = bfr(x[i] + acc);
      }
    }
    free(logits); free(ids); free(wts); free(pe); free(pr); free(fill); free(used); free(xsp); free(hsp); free(hb); free(ys);
  } else {                                                                      /* :149-152 */
    const int I = c->I;
    float* hb = (float*)malloc(sizeof(float) * (size_t)n * I);
#pragma omp parallel
    {
      float* wg = (float*)malloc(sizeof(float) * (size_t)H * 2);
      float* wu = wg + H;
#pragma omp for schedule(dynamic, 8)
      for (int j = 0; j < I; ++j) {
        const float sg = row_f32(&y->wgu, wt, (size_t)(2 * j), H, wg);
        const float su = row_f32(&y->wgu, wt, (size_t)(2 * j + 1), H, wu);
        for (int b = 0; b < n; ++b) {
          const float* xb = xs + (size_t)b * H;
          const float g = bfr(row_dot(wg, sg, wt, xb, H));
          const float up = bfr(row_dot(wu, su, wt, xb, H));
          hb[(size_t)b * I + j] = bfr(bfr(silu(g)) * up);
        }
      }
      free(wg);
    }
    gemv_rows_multi(&y->wd, wt, H, I, hb, I, n, t, H);
    for (size_t i = 0; i < (size_t)n * H; ++i) X[i] = bfr(X[i] + t[i]);
    free(hb);
  }
  free(xs); free(qkv); free(o); free(t);
}

/* n rows: row r is sequence seqs[r]'s step with input token toks[r] at position pos[r]; its greedy token into out[r]
 * (each equal to orc_step_seq of that row given the cache its earlier positions left).  Rows of one sequence must hold
 * distinct positions; a row attends to every position of its sequence up to its own, including the positions of the
 * other rows.  dump_x [n][L][H] residual after each layer, dump_ids / dump_wts [n][L][TOPK]; each may be NULL. */
EXPORT int orc_step_rows(void* h, int n, const int32_t* seqs, const int32_t* toks, const int32_t* pos, int32_t* out,
                         float* dump_x, int32_t* dump_ids, float* dump_wts) {
  orc_model* m = (orc_model*)h; const orc_config* c = &m->c;
  if (c->arch != 0 || n < 1) return 1;
  const int H = c->H, V = c->V, L = c->L, K = c->TOPK > 0 ? c->TOPK : 1;
  orc_row* rows = (orc_row*)malloc(sizeof(orc_row) * (size_t)n);
  for (int r = 0; r < n; ++r) {
    if (seqs[r] < 0 || seqs[r] >= m->batch || pos[r] < 0 || pos[r] >= c->max_ctx || toks[r] < 0 || toks[r] >= V) {
      free(rows);
      return 1;
    }
    rows[r].bt = m->btab + (size_t)seqs[r] * m->nbps;
    rows[r].pos = pos[r];
  }
  float* X = (float*)malloc(sizeof(float) * (size_t)n * H);
  for (int b = 0; b < n; ++b)
    for (int i = 0; i < H; ++i) X[(size_t)b * H + i] = bf2f(m->embed[(size_t)toks[b] * H + i]);
  for (int l = 0; l < L; ++l) {
    layer_rows(m, l, X, n, rows, dump_ids ? dump_ids + (size_t)l * K : NULL, dump_wts ? dump_wts + (size_t)l * K : NULL,
               L * K);
    if (dump_x)
      for (int b = 0; b < n; ++b) memcpy(dump_x + ((size_t)b * L + l) * H, X + (size_t)b * H, sizeof(float) * (size_t)H);
  }
  float* xs = (float*)malloc(sizeof(float) * (size_t)n * H);
  for (int b = 0; b < n; ++b) rmsnorm(X + (size_t)b * H, NULL, H, c->eps, xs + (size_t)b * H);   /* :155 */
  /* lm_head rows against every row's vector, argmax (first maximum) per row, rows split over the threads */
  const int nt = omp_get_max_threads();
  float* bv = (float*)malloc(sizeof(float) * (size_t)nt * n);
  int* bi = (int*)malloc(sizeof(int) * (size_t)nt * n);
  int16_t* xsp = NULL;                             /* matrix-core order: the rows' vectors decomposed once */
  if (m->mfma) {
    xsp = (int16_t*)malloc(sizeof(int16_t) * 2 * (size_t)n * H);
    for (int b = 0; b < n; ++b) mfma_split_row(xs + (size_t)b * H, H, xsp + 2 * (size_t)b * H, xsp + (2 * (size_t)b + 1) * H);
  }
#pragma omp parallel
  {
    const int tid = omp_get_thread_num(), nth = omp_get_num_threads();
    float* wf = (float*)malloc(sizeof(float) * (size_t)H * ORC_TR);
    int16_t* wsp = xsp ? (int16_t*)malloc(sizeof(int16_t) * 2 * (size_t)H * ORC_TR) : NULL;
    for (int b = 0; b < n; ++b) { bv[(size_t)tid * n + b] = -INFINITY; bi[(size_t)tid * n + b] = -1; }
    const int r0 = (int)((int64_t)V * tid / nth), r1 = (int)((int64_t)V * (tid + 1) / nth);
    const orc_mat lm = {m->lm_head, NULL, NULL};
    for (int rt = r0; rt < r1; rt += ORC_TR) {                                  /* :157-158 */
      const int nr = r1 - rt < ORC_TR ? r1 - rt : ORC_TR;
      for (int i = 0; i < nr; ++i) {
        row_f32(&lm, 0, (size_t)(rt + i), H, wf + (size_t)i * H);
        if (wsp) mfma_split_row(wf + (size_t)i * H, H, wsp + 2 * (size_t)i * H, wsp + (2 * (size_t)i + 1) * H);
      }
      for (int b = 0; b < n; ++b)
        for (int i = 0; i < nr; ++i) {                /* rows ascending within the thread's range */
          const float v = wsp ? bfr(mfma_dot_split(wsp + 2 * (size_t)i * H, wsp + (2 * (size_t)i + 1) * H,
                                                   xsp + 2 * (size_t)b * H, xsp + (2 * (size_t)b + 1) * H, H))
                              : bfr(dot64f(wf + (size_t)i * H, xs + (size_t)b * H, H));
          if (bi[(size_t)tid * n + b] < 0 || v > bv[(size_t)tid * n + b]) { bv[(size_t)tid * n + b] = v; bi[(size_t)tid * n + b] = rt + i; }
        }
    }
    free(wf); free(wsp);
  }
  free(xsp);
  for (int b = 0; b < n; ++b) {                    /* threads hold ascending row ranges: the first maximum wins */
    int best = -1; float v = -INFINITY;
    for (int t = 0; t < nt; ++t) {
      const int i = bi[(size_t)t * n + b];
      if (i >= 0 && (best < 0 || bv[(size_t)t * n + b] > v)) { v = bv[(size_t)t * n + b]; best = i; }
    }
    out[b] = best < 0 ? 0 : best;
  }
  free(rows); free(X); free(xs); free(bv); free(bi);
  return 0;
}

/* positions pos0 .. pos0+n-1 of sequence `seq` with input tokens toks[0..n): n rows of one sequence */
EXPORT int orc_prefill_seq(void* h, int seq, const int32_t* toks, int pos0, int n, int32_t* out) {
  if (n < 1) return 1;
  int32_t* seqs = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
  int32_t* pos = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
  for (int b = 0; b < n; ++b) { seqs[b] = seq; pos[b] = pos0 + b; }
  const int r = orc_step_rows(h, n, seqs, toks, pos, out, NULL, NULL, NULL);
  free(seqs);
  free(pos);
  return r;
}

/* ref_numpy.py:105-158 Ref.step for sequence `seq` of the batch: token at position pos -> greedy next token.
 * The sequences of a batch share the weights and nothing else, so a batched step is this, once per sequence.
 * dump_x [L][H] residual after each layer; dump_ids/dump_wts [L][TOPK]; each may be NULL. */
static void mla_layer_step(orc_model* m, int l, float* x, int pos, const int32_t* bt, int32_t* ids_out, float* wts_out,
                           float* logits_out);

EXPORT int32_t orc_step_seq(void* h, int seq, int32_t tok, int pos, float* dump_x, int32_t* dump_ids, float* dump_wts) {
  orc_model* m = (orc_model*)h; const orc_config* c = &m->c;
  const int H = c->H;
  const int32_t* bt = m->btab + (size_t)seq * m->nbps;
  float* x = (float*)malloc(sizeof(float) * (size_t)H);
  for (int i = 0; i < H; ++i) x[i] = bf2f(m->embed[(size_t)tok * H + i]);
  for (int l = 0; l < c->L; ++l) {
    (c->arch == 1 ? mla_layer_step : layer_step)(m, l, x, pos, bt, dump_ids ? dump_ids + (size_t)l * c->TOPK : NULL,
                                                   dump_wts ? dump_wts + (size_t)l * c->TOPK : NULL, NULL);
    if (dump_x) memcpy(dump_x + (size_t)l * H, x, sizeof(float) * (size_t)H);
  }
  float* xs = (float*)malloc(sizeof(float) * (size_t)H);
  rmsnorm(x, NULL, H, c->eps, xs);                                  /* :155 final norm (weight 1.0) */
  const int V = c->V;
  float* lg = (float*)malloc(sizeof(float) * (size_t)V);
  if (m->mfma) {                                                     /* :157 */
    const orc_mat lm = {m->lm_head, NULL, NULL};
#pragma omp parallel for schedule(static)
    for (int v = 0; v < V; ++v) lg[v] = bfr(gateup_dot(m, &lm, 0, (size_t)v, xs, H));
  } else {
    gemv_bf(m->lm_head, V, H, xs, lg);
  }
  int best = 0;
  for (int v = 1; v < V; ++v) if (lg[v] > lg[best]) best = v;        /* :158 first maximum */
  free(x); free(xs); free(lg);
  return best;
}
EXPORT int32_t orc_step(void* h, int32_t tok, int pos, float* dump_x, int32_t* dump_ids, float* dump_wts) {
  return orc_step_seq(h, 0, tok, pos, dump_x, dump_ids, dump_wts);
}

/* the single-layer configuration: run layer `l` on the given residual x (in place) at position pos */
EXPORT void orc_layer_step_seq(void* h, int seq, int l, float* x, int pos, int32_t* ids_out, float* wts_out,
                               float* logits_out) {
  orc_model* m = (orc_model*)h;
  (m->c.arch == 1 ? mla_layer_step : layer_step)(m, l, x, pos, m->btab + (size_t)seq * m->nbps, ids_out, wts_out,
                                                 logits_out);
}
EXPORT void orc_layer_step(void* h, int l, float* x, int pos, int32_t* ids_out, float* wts_out, float* logits_out) {
  orc_layer_step_seq(h, 0, l, x, pos, ids_out, wts_out, logits_out);
}

/* generate every expert of every layer now (so that timing excludes generation) */
EXPORT void orc_materialize_experts(void* h) {
  orc_model* m = (orc_model*)h;
  if (!m->c.moe) return;
  for (int l = 0; l < m->c.L; ++l)
    for (int e = 0; e < m->c.E; ++e) ensure_expert(m, l, e);
}

static const orc_mat* mat_of(orc_model* m, int kind, int l, int e) {
  switch (kind) {
    case S_WQKV: return &m->ly[l].wqkv;
    case S_WO: return &m->ly[l].wo;
    case S_W13: ensure_expert(m, l, e); return &m->ly[l].w13[e];
    case S_W2: ensure_expert(m, l, e); return &m->ly[l].w2[e];
    case S_WGU: return &m->ly[l].wgu;
    case S_WD: return &m->ly[l].wd;
    case S_WSGU: return &m->ly[l].wsgu;
    case S_WSD: return &m->ly[l].wsd;
    default: return NULL;
  }
}
/* raw weight access for tests (natural layout); expert tensors are generated on first use.  bf16 rows (NULL for
 * a matrix held as fp8), or the e4m3 rows and per-row scales of an fp8 matrix (NULL otherwise). */
EXPORT const uint16_t* orc_weight(void* h, int kind, int l, int e) {
  orc_model* m = (orc_model*)h;
  switch (kind) {
    case S_EMBED: return m->embed;
    case S_LMHEAD: return m->lm_head;
    case S_ROUTER: return m->ly[l].wr;
    case S_WKVB: return m->ly[l].wkvb;
    default: { const orc_mat* w = mat_of(m, kind, l, e); return w ? w->w : NULL; }
  }
}
EXPORT const uint8_t* orc_weight_q(void* h, int kind, int l, int e) {
  const orc_mat* w = mat_of((orc_model*)h, kind, l, e);
  return w ? w->q : NULL;
}
EXPORT const float* orc_weight_scale(void* h, int kind, int l, int e) {
  const orc_mat* w = mat_of((orc_model*)h, kind, l, e);
  return w ? w->s : NULL;
}
EXPORT int orc_num_threads(void) { return omp_get_max_threads(); }

/* ================================================================== DeepSeek-V2 (arch 1) */
/* yarn_get_mscale (reference_decode.py:78-83) */
static double yarn_mscale(double scale, double mscale) { return scale <= 1.0 ? 1.0 : 0.1 * mscale * log(scale) + 1.0; }

/* DeepseekV2YarnRotaryEmbedding tables (reference_decode.py:85-118) in the float32 steps the reference's numpy takes:
 * correction range in float64, ramp / mask / frequencies / products in float32, then cos and sin (libm) times the
 * mscale ratio (1.0 when mscale == mscale_all_dim).  Only the first half is stored (emb = cat(freqs, freqs)). */
EXPORT void orc_yarn_tables(const orc_config* c, int ctx, float* cs, float* sn) {
  const int dim = c->qk_rope, half = dim / 2;
  const double base = c->theta, two_pi = 2.0 * 3.141592653589793;
  const double lowd = (dim * log(c->rope_orig_max / (c->beta_fast * two_pi))) / (2.0 * log(base));
  const double highd = (dim * log(c->rope_orig_max / (c->beta_slow * two_pi))) / (2.0 * log(base));
  int low = (int)floor(lowd), high = (int)ceil(highd);
  if (low < 0) low = 0;
  if (high > dim - 1) high = dim - 1;
  const float span = low == high ? (float)((double)high + 0.001 - (double)low) : (float)(high - low);
  const float ms = (float)(yarn_mscale(c->rope_factor, c->rope_mscale) / yarn_mscale(c->rope_factor, c->rope_mscale_all));
  float inv[256];
  for (int i = 0; i < half; ++i) {
    const float e = (float)(2 * i) / (float)dim;
    const float pw = powf((float)base, e);
    const float extra = 1.0f / pw, inter = 1.0f / ((float)c->rope_factor * pw);
    float ramp = ((float)i - (float)low) / span;
    ramp = ramp < 0.0f ? 0.0f : ramp > 1.0f ? 1.0f : ramp;
    const float mask = 1.0f - ramp;
    inv[i] = inter * (1.0f - mask) + extra * mask;
  }
  for (int t = 0; t < ctx; ++t)
    for (int i = 0; i < half; ++i) {
      const float f = (float)t * inv[i];
      cs[(size_t)t * half + i] = cosf(f) * ms;
      sn[(size_t)t * half + i] = sinf(f) * ms;
    }
}

/* DeepSeek-V2 RoPE (reference_decode.py:120-136): de-interleave (x0, x2, ..., x1, x3, ...), then rotate_half:
 * out[i] = x[2i] c_i - x[2i+1] s_i, out[i + d/2] = x[2i+1] c_i + x[2i] s_i, each product and sum in fp32; bfr after */
static void rope_ds(const float* x, int d, const float* cs, const float* sn, float* out) {
  const int half = d / 2;
  for (int i = 0; i < half; ++i) {
    const float a = x[2 * i], b = x[2 * i + 1];
    out[i] = bfr(a * cs[i] + (-b) * sn[i]);
    out[i + half] = bfr(b * cs[i] + a * sn[i]);
  }
}
EXPORT void orc_rope_ds(const float* x, int d, const float* cs, const float* sn, float* out) { rope_ds(x, d, cs, sn, out); }

static void* mla_model_create(orc_model* m) {
  const orc_config* c = &m->c;
  const uint64_t seed = m->seed;
  const float ws = m->scale;
  const int NH = c->NH, QD = c->qk_nope + c->qk_rope, KVL = c->kv_lora, CD = mla_cache_dim(c);
  const int NQA = NH * QD + KVL + c->qk_rope;
  m->embed = gen_tensor(seed, sid(S_EMBED, -1, 0), (size_t)c->V * c->H, ws);
  m->lm_head = gen_tensor(seed, sid(S_LMHEAD, -1, 0), (size_t)c->V * c->H, ws);
  m->batch = c->batch > 1 ? c->batch : 1;
  m->nbps = (c->max_ctx + c->block_size - 1) / c->block_size;
  m->nblocks = m->batch * m->nbps;
  m->btab = (int32_t*)malloc(sizeof(int32_t) * (size_t)m->nblocks);
  for (int i = 0; i < m->nblocks; ++i) m->btab[i] = i;
  m->ly = (orc_layer*)calloc((size_t)c->L, sizeof(orc_layer));
  for (int l = 0; l < c->L; ++l) {
    orc_layer* y = &m->ly[l];
    y->wqkv = gen_mat(seed, sid(S_WQKV, l, 0), (size_t)NQA, c->H, ws, c->wdtype);
    y->wo = gen_mat(seed, sid(S_WO, l, 0), (size_t)c->H, NH * c->v_head, ws, c->wdtype);
    y->wkvb = gen_tensor(seed, sid(S_WKVB, l, 0), (size_t)NH * (c->qk_nope + c->v_head) * KVL, ws);
    if (l < c->first_dense) {
      y->wgu = gen_mat(seed, sid(S_WGU, l, 0), (size_t)2 * c->dense_I, c->H, ws, c->wdtype);
      y->wd = gen_mat(seed, sid(S_WD, l, 0), (size_t)c->H, c->dense_I, ws, c->wdtype);
    } else {
      y->wr = gen_tensor(seed, sid(S_ROUTER, l, 0), (size_t)c->E * c->H, ws);
      y->w13 = (orc_mat*)calloc((size_t)c->E, sizeof(orc_mat));
      y->w2 = (orc_mat*)calloc((size_t)c->E, sizeof(orc_mat));
      y->wsgu = gen_mat(seed, sid(S_WSGU, l, 0), (size_t)2 * c->n_shared * c->MI, c->H, ws, c->wdtype);
      y->wsd = gen_mat(seed, sid(S_WSD, l, 0), (size_t)c->H, c->n_shared * c->MI, ws, c->wdtype);
    }
    y->kc = (uint16_t*)calloc((size_t)m->nblocks * c->block_size * CD, sizeof(uint16_t));
  }
  const int half = c->qk_rope / 2;
  m->rcos = (float*)malloc(sizeof(float) * (size_t)c->max_ctx * half);
  m->rsin = (float*)malloc(sizeof(float) * (size_t)c->max_ctx * half);
  orc_yarn_tables(c, c->max_ctx, m->rcos, m->rsin);
  /* softmax_scale (reference_decode.py:198-206): q_head_dim^-0.5 * mscale_all^2, applied as fp32 */
  const double mm = yarn_mscale(c->rope_factor, c->rope_mscale_all);
  m->attn_scale = (float)(pow((double)QD, -0.5) * mm * mm);
  return m;
}
EXPORT float orc_attn_scale(void* h) { return ((orc_model*)h)->attn_scale; }

/* canonical dot of a row zero-padded to a multiple of 128 elements (the device stores such rows padded): one more
 * fma(0, 0, acc) per lane when K % 128 == 64 */
static inline float dot64_pad(const orc_mat* m, int wdtype, size_t r, const float* x, int K) {
  if (K % 128 == 0) return mat_dot(m, wdtype, r, x, K);
  float acc[64];
  for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
  for (int k0 = 0; k0 < K; k0 += 64)
    for (int l = 0; l < 64; ++l) {
      const float w = wdtype == 0 ? bf2f(m->w[r * K + k0 + l]) : e4m3_f(m->q[r * K + k0 + l]);
      acc[l] = fmaf(w, x[k0 + l], acc[l]);
    }
  for (int l = 0; l < 64; ++l) acc[l] = fmaf(0.0f, 0.0f, acc[l]);
  const float d = butterfly64(acc);
  return wdtype == 0 ? d : d * m->s[r];
}

/* one MLA head over positions 0..n-1 of the latent cache (reference_decode.py:250-253 in chunked form):
 * s_t = ((q_c . c_t over kv_lora, ascending fma) + (q_pe . kpe_t over qk_rope, ascending fma)) * scale; chunks of 64
 * with m_c, p = expf(s - m_c), l_c and a_c[i] = sum_t p_t c_t[i] as ascending fma chains; merge as attention_head;
 * o_c = A / L in fp32 (not rounded: the reference keeps o_c fp32 into W_UV) */
static void mla_head(const float* q_c, const float* q_pe, const uint16_t* kc, const int32_t* bt, int n, int KVL, int R,
                     int BS, float scale, float* o_c) {
  const int CD = KVL + R;
  float A[1024], a[1024], mc[256];
  float L = 0.0f, M = -INFINITY;
  const int nch = (n + ATT_CHUNK - 1) / ATT_CHUNK;
  float* sc = (float*)malloc(sizeof(float) * (size_t)n);
  for (int t = 0; t < n; ++t) {
    const int blk = bt[t / BS], off = t % BS;
    float s1 = 0.0f, s2 = 0.0f;
    for (int i = 0; i < KVL; ++i) s1 = fmaf(q_c[i], bf2f(kc[kv_k_index(blk, off, 0, i, 1, CD, BS)]), s1);
    for (int j = 0; j < R; ++j) s2 = fmaf(q_pe[j], bf2f(kc[kv_k_index(blk, off, 0, KVL + j, 1, CD, BS)]), s2);
    sc[t] = (s1 + s2) * scale;
  }
  for (int c = 0; c < nch; ++c) {
    float m = -INFINITY;
    for (int t = c * ATT_CHUNK; t < n && t < (c + 1) * ATT_CHUNK; ++t) if (sc[t] > m) m = sc[t];
    mc[c] = m;
    if (m > M) M = m;
  }
  for (int i = 0; i < KVL; ++i) A[i] = 0.0f;
  for (int c = 0; c < nch; ++c) {
    float l = 0.0f;
    for (int i = 0; i < KVL; ++i) a[i] = 0.0f;
    for (int t = c * ATT_CHUNK; t < n && t < (c + 1) * ATT_CHUNK; ++t) {
      const int blk = bt[t / BS], off = t % BS;
      const float p = mk_expf(sc[t] - mc[c]);
      l = l + p;
      for (int i = 0; i < KVL; ++i) a[i] = fmaf(p, bf2f(kc[kv_k_index(blk, off, 0, i, 1, CD, BS)]), a[i]);
    }
    const float w = mk_expf(mc[c] - M);
    L = fmaf(w, l, L);
    for (int i = 0; i < KVL; ++i) A[i] = fmaf(w, a[i], A[i]);
  }
  for (int i = 0; i < KVL; ++i) o_c[i] = A[i] / L;
  free(sc);
}

/* the router of DeepSeek-V2 (reference_decode.py:271-278): fp32 softmax of the fp32 logits, top-k by probability
 * (ties to the lower id), weights = probability * routed_scale (or renormalised when norm_topk), kept in fp32 */
static void route_ds(const float* logits, int E, int K, int renorm, float rscale, int32_t* ids, float* wts) {
  float M = -INFINITY;
  for (int e = 0; e < E; ++e) if (logits[e] > M) M = logits[e];
  float p[1024];
  for (int e = 0; e < E; ++e) p[e] = mk_expf(logits[e] - M);
  const float S = sum64(p, E);
  for (int e = 0; e < E; ++e) p[e] = p[e] / S;
  unsigned char taken[1024] = {0};
  float sel = 0.0f, wv[64];
  for (int k = 0; k < K; ++k) {
    int bi = -1; float bv = -1.0f;
    for (int e = 0; e < E; ++e) if (!taken[e] && p[e] > bv) { bv = p[e]; bi = e; }
    taken[bi] = 1; ids[k] = bi; wv[k] = bv; sel = sel + bv;
  }
  for (int k = 0; k < K; ++k) wts[k] = renorm ? wv[k] / (sel + 1e-20f) : wv[k] * rscale;
}
EXPORT void orc_route_ds(const float* logits, int E, int K, int renorm, float rscale, int32_t* ids, float* wts) {
  route_ds(logits, E, K, renorm, rscale, ids, wts);
}

/* one DeepSeek-V2 decoder layer (reference_decode.py:294-302) at position pos on residual x (in place) */
static void mla_layer_step(orc_model* m, int l, float* x, int pos, const int32_t* bt, int32_t* ids_out, float* wts_out,
                           float* logits_out) {
  const orc_config* c = &m->c;
  orc_layer* y = &m->ly[l];
  const int H = c->H, NH = c->NH, NOPE = c->qk_nope, R = c->qk_rope, VH = c->v_head, KVL = c->kv_lora, BS = c->block_size;
  const int QD = NOPE + R, NQA = NH * QD + KVL + R, CD = KVL + R, wt = c->wdtype;
  const int W = H > c->dense_I ? H : c->dense_I;
  float* xs = (float*)malloc(sizeof(float) * (size_t)(W + 128));
  float* qa = (float*)malloc(sizeof(float) * (size_t)NQA);
  float* out = (float*)malloc(sizeof(float) * (size_t)NH * VH);
  float* t = (float*)malloc(sizeof(float) * (size_t)H);
  rmsnorm(x, NULL, H, c->eps, xs);                                  /* :222 input_layernorm (weight 1.0) */
  gemv_mat(&y->wqkv, wt, NQA, H, xs, qa);                           /* :225, :229 q_proj, kv_a_proj (bf16) */
  const float* cs = m->rcos + (size_t)pos * (R / 2);
  const float* sn = m->rsin + (size_t)pos * (R / 2);
  float cnew[1024], kpe[256];
  rmsnorm(qa + NH * QD, NULL, KVL, c->eps, cnew);                   /* :231 kv_a_layernorm (weight 1.0) */
  rope_ds(qa + NH * QD + KVL, R, cs, sn, kpe);                      /* :234 */
  const int blk = bt[pos / BS], off = pos % BS;                     /* :236-237 append the latent row */
  for (int i = 0; i < KVL; ++i) y->kc[kv_k_index(blk, off, 0, i, 1, CD, BS)] = f2bf(cnew[i]);
  for (int j = 0; j < R; ++j) y->kc[kv_k_index(blk, off, 0, KVL + j, 1, CD, BS)] = f2bf(kpe[j]);
#pragma omp parallel for schedule(static)
  for (int h = 0; h < NH; ++h) {                                    /* :245-254 per head, absorbed */
    const float* q = qa + (size_t)h * QD;
    float qpe[256], q_c[1024], o_c[1024];
    rope_ds(q + NOPE, R, cs, sn, qpe);                               /* :235 */
    /* q_c[i] = sum_d q_nope[d] * W_UK[h][d][i]: the canonical dot of column i of W_UK (kv_b rows h*(NOPE+VH)+d) */
    const uint16_t* wuk = y->wkvb + (size_t)h * (NOPE + VH) * KVL;
    for (int i = 0; i < KVL; ++i) {
      uint16_t colb[512];
      for (int d = 0; d < NOPE; ++d) colb[d] = wuk[(size_t)d * KVL + i];
      q_c[i] = dot64(colb, q, NOPE);
    }
    mla_head(q_c, qpe, y->kc, bt, pos + 1, KVL, R, BS, m->attn_scale, o_c);
    const uint16_t* wuv = wuk + (size_t)NOPE * KVL;                  /* :254 out[h] = W_UV o_c, bf16 at :256 */
    for (int d = 0; d < VH; ++d) out[(size_t)h * VH + d] = bfr(dot64(wuv + (size_t)d * KVL, o_c, KVL));
  }
  gemv_mat(&y->wo, wt, H, NH * VH, out, t);                         /* :256 o_proj, bf16 */
  for (int i = 0; i < H; ++i) x[i] = bfr(x[i] + t[i]);              /* :300 residual */
  rmsnorm(x, NULL, H, c->eps, xs);                                  /* :301 post_attention_layernorm */
  if (l < c->first_dense) {                                         /* :290-291 dense MLP */
    const int I = c->dense_I, IP = (I + 127) / 128 * 128;
    float* hb = (float*)calloc((size_t)IP, sizeof(float));
#pragma omp parallel for schedule(static)
    for (int j = 0; j < I; ++j) {
      const float g = bfr(mat_dot(&y->wgu, wt, (size_t)(2 * j), xs, H));
      const float u = bfr(mat_dot(&y->wgu, wt, (size_t)(2 * j + 1), xs, H));
      hb[j] = bfr(bfr(silu(g)) * u);
    }
#pragma omp parallel for schedule(static)
    for (int i = 0; i < H; ++i) t[i] = bfr(dot64_pad(&y->wd, wt, (size_t)i, hb, I));
    for (int i = 0; i < H; ++i) x[i] = bfr(x[i] + t[i]);
    free(hb);
  } else {                                                          /* :268-287 MoE */
    const int E = c->E, K = c->TOPK, MI = c->MI, SI = c->n_shared * MI;
    float logits[1024];
#pragma omp parallel for schedule(static)
    for (int e = 0; e < E; ++e) logits[e] = dot64(y->wr + (size_t)e * H, xs, H);   /* :271 fp32 router, not rounded */
    if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t)E);
    int32_t ids[64]; float wts[64];
    route_ds(logits, E, K, c->norm_topk, c->routed_scale, ids, wts);
    if (ids_out) memcpy(ids_out, ids, sizeof(int32_t) * (size_t)K);
    if (wts_out) memcpy(wts_out, wts, sizeof(float) * (size_t)K);
    for (int k = 0; k < K; ++k) ensure_expert(m, l, ids[k]);
    int order[64];                                                  /* y summed in ascending expert id */
    for (int k = 0; k < K; ++k) order[k] = k;
    for (int a = 1; a < K; ++a)
      for (int b = a; b > 0 && ids[order[b]] < ids[order[b - 1]]; --b) { int q = order[b]; order[b] = order[b - 1]; order[b - 1] = q; }
    float* hk = (float*)malloc(sizeof(float) * (size_t)(SI > MI ? SI : MI));
    float* ys = (float*)malloc(sizeof(float) * (size_t)K * H);
    for (int k = 0; k < K; ++k) {                                   /* :281-284, mlp_unit :259-265 */
      const orc_mat* W13 = &y->w13[ids[k]];
#pragma omp parallel for schedule(static)
      for (int j = 0; j < MI; ++j) {
        const float g = bfr(mat_dot(W13, wt, (size_t)(2 * j), xs, H));
        const float u = bfr(mat_dot(W13, wt, (size_t)(2 * j + 1), xs, H));
        hk[j] = bfr(bfr(silu(g)) * u);
      }
      const orc_mat* W2 = &y->w2[ids[k]];
#pragma omp parallel for schedule(static)
      for (int i = 0; i < H; ++i) ys[(size_t)k * H + i] = bfr(wts[k] * bfr(dot64_pad(W2, wt, (size_t)i, hk, MI)));
    }
#pragma omp parallel for schedule(static)
    for (int j = 0; j < SI; ++j) {                                  /* :286 shared experts */
      const float g = bfr(mat_dot(&y->wsgu, wt, (size_t)(2 * j), xs, H));
      const float u = bfr(mat_dot(&y->wsgu, wt, (size_t)(2 * j + 1), xs, H));
      hk[j] = bfr(bfr(silu(g)) * u);
    }
#pragma omp parallel for schedule(static)
    for (int i = 0; i < H; ++i) {
      float acc = 0.0f;                                             /* :280-284 fp32 sum of the rounded terms */
      for (int k = 0; k < K; ++k) acc = acc + ys[(size_t)order[k] * H + i];
      const float sh = bfr(dot64_pad(&y->wsd, wt, (size_t)i, hk, SI));
      t[i] = bfr(bfr(acc) + sh);                                    /* :287 */
    }
    for (int i = 0; i < H; ++i) x[i] = bfr(x[i] + t[i]);            /* :302 */
    free(hk); free(ys);
  }
  free(xs); free(qa); free(out); free(t);
}

/* fill positions [0, n) of sequence seq's latent cache in every layer with bf16 N(0,1): element (t, i) is number
 * t*CD + i of the layer's stream (kind 10) for that sequence */
EXPORT void orc_fill_latent_random_seq(void* h, int seq, int n) {
  orc_model* m = (orc_model*)h; const orc_config* c = &m->c;
  const int CD = mla_cache_dim(c), BS = c->block_size;
  const int32_t* bt = m->btab + (size_t)seq * m->nbps;
  for (int l = 0; l < c->L; ++l) {
    const uint64_t kk = stream_key(m->seed, sid(S_KINIT, l, seq));
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n; ++t)
      for (int i = 0; i < CD; ++i)
        m->ly[l].kc[kv_k_index(bt[t / BS], t % BS, 0, i, 1, CD, BS)] = f2bf(mk_normal(kk, (uint64_t)t * CD + i));
  }
}
