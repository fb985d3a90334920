#pragma once
// Batch-small decode step for gfx950 (MI355X): one persistent cooperative launch per token that runs every
// layer's phases back to back with grid barriers, or (unfused mode) one ordinary launch per phase with the
// same device functions.
//
// Reference path (relative to the reference checkout): examples/llm/ref_numpy.py:105-158 is the numerical
// specification; examples/llm/tiles.hip:23-357 and etx/codegen/kernel.py:471-605 are the tile bodies and
// the persistent worker loop this file replaces.
//
// Phases of one layer (MoE):   P1 norm + QKV GEMV | P2 q/k norm, RoPE, paged KV append, attention |
//                              P3 O projection + residual | P4 norm + router GEMV |
//                              P5 top-k + expert gate/up GEMV + SiLU*up | P6 expert down GEMV, weight, combine, residual
// Dense layers replace P4-P6 by gate/up (+SiLU*up) and down (+residual).  Head: final norm + lm_head GEMV with
// a 64-bit packed argmax key, then the token write.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include "etxmk.h"
#include "mk_numerics.h"

namespace mk {

constexpr int NT = 512;                 // threads per workgroup: 8 waves, two per SIMD
constexpr int NWAVE = NT / 64;
constexpr int CHUNK = 64;               // attention positions per chunk
constexpr int HDIM = 128;               // head dim handled by the attention phase
constexpr int MAX_H = 4096;
constexpr int MAX_K = 12288;
constexpr int MAX_CTX = 4096;
constexpr int MAX_E = 256;
constexpr int MAX_TOPK = 8;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct LayerW {
  const uint16_t *ln1, *ln2, *qn, *kn;
  const uint16_t *wqkv, *wo, *wr, *w13, *w2, *wgu, *wd;
  uint16_t *kc, *vc;
};

struct Params {
  int H, NH, NKV, HD, I, E, TOPK, MI, L, V;
  int moe, qk_norm, norm_topk, BS, max_ctx, nblocks;
  float eps, attn_scale;
  const uint16_t* embed;
  const uint16_t* lm_head;
  const uint16_t* final_norm;
  const LayerW* layers;
  const float* rope_cos;
  const float* rope_sin;
  const int32_t* btab;
  float* x;
  float* qkv;
  float* o;
  float* logits;
  float* hbuf;
  uint64_t* amax;
  uint32_t* bar;
  int32_t* abort_word;
  int32_t* tokens;
  int32_t* out_tokens;
  float* dump_x;
  int32_t* dump_ids;
  float* dump_wts;
  float* dump_logits;
  int pos, write_next, l0, l1, do_embed, do_head;
  uint32_t bar_base;
  int nwg;
  uint64_t spin_ticks;
};

struct Smem {
  union {
    struct {
      float xf[MAX_H];                  // residual (natural order, fp32)
      alignas(16) uint16_t xs[MAX_K];   // GEMV input vector, lane-permuted bf16
    } g;
    struct {
      float q[HDIM], k[HDIM], v[HDIM];
      float p[MAX_CTX];                 // exp(s - m_c) per position
      float mc[MAX_CTX / CHUNK];
      float lc[MAX_CTX / CHUNK];
      float ac[MAX_CTX / CHUNK][HDIM];
    } a;
  };
  float rs;
  int32_t ids[MAX_TOPK];
  float wts[MAX_TOPK];
  int32_t order[MAX_TOPK];
  float prob[MAX_E];
  int32_t abort;
};

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// ---------------------------------------------------------------- grid barrier
// Monotonic counters (never reset): barrier k of this launch is generation gen = gen_base + k + 1.
// Arrival is hierarchical to spread the atomics over 8 lines: workgroup w counts into group w % 8; the last
// arrival of a group counts into the global word; the last group's last arrival writes the generation into
// the 8 release flags, and every workgroup polls its group's flag.
// Visibility: every value another workgroup reads is written with an agent-scope (sc1) store and read with an
// agent-scope load; each wave waits for its own stores to complete (s_waitcnt 0) before the workgroup barrier
// that precedes the arrival, so no L2 write-back or invalidate is needed.  The wait is bounded by a wall-clock
// limit; on expiry the abort word is set and every workgroup leaves.
__device__ __forceinline__ bool grid_sync(const Params& p, int& k, Smem& s) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int g = blockIdx.x & 7;
    const uint32_t ng = (uint32_t)(p.nwg - g + 7) / 8u;
    const uint32_t gen = p.bar_base + (uint32_t)k + 1u;
    uint32_t* grp = p.bar + 64 * g;
    const uint32_t old = __hip_atomic_fetch_add(grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old + 1u == gen * ng) {
      const uint32_t o2 = __hip_atomic_fetch_add(p.bar + 64 * 8, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (o2 + 1u == gen * 8u)
        for (int j = 0; j < 8; ++j) __hip_atomic_store(p.bar + 64 * (9 + j), gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const uint32_t* flag = p.bar + 64 * (9 + g);
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    int ab = 0;
    uint32_t polls = 0;
    while ((int32_t)(__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - gen) < 0) {
      __builtin_amdgcn_s_sleep(1);
      if ((++polls & 255u) == 0) {
        if (ld_ag_i(p.abort_word) != 0) { ab = 1; break; }
        if (__builtin_amdgcn_s_memrealtime() - t0 > p.spin_ticks) {
          st_ag_i(p.abort_word, 2);
          ab = 1;
          break;
        }
      }
    }
    s.abort = ab;
  }
  __syncthreads();
  ++k;
  return s.abort == 0;
}

// ---------------------------------------------------------------- vectors into LDS
// x (fp32 global, or the bf16 embedding row for the first layer) -> s.g.xf; normed and lane-permuted -> s.g.xs.
// ref_numpy.py:71-73: r = 1/sqrt(mean(x^2) + eps), out = bfr(w * bfr(x * r)); the sum of squares in dot order.
__device__ __forceinline__ void build_norm_x(const Params& p, const float* xg, const uint16_t* xrow, const uint16_t* w, Smem& s) {
  const int H = p.H;
  if (xrow) {
    for (int i = threadIdx.x; i < H; i += NT) s.g.xf[i] = bf2f(xrow[i]);
  } else {
    for (int i = threadIdx.x; i < H / 2; i += NT) {
      const uint64_t u = ld_ag64((const uint64_t*)xg + i);
      s.g.xf[2 * i] = bits2f((uint32_t)u);
      s.g.xf[2 * i + 1] = bits2f((uint32_t)(u >> 32));
    }
  }
  __syncthreads();
  if (wave_id() == 0) {
    float acc = 0.0f;
    for (int k = lane_id(); k < H; k += 64) acc = __builtin_fmaf(s.g.xf[k], s.g.xf[k], acc);
    acc = wave_sum_xor(acc);
    if (lane_id() == 0) s.rs = 1.0f / __builtin_sqrtf(acc / (float)H + p.eps);
  }
  __syncthreads();
  const float r = s.rs;
  for (int q = threadIdx.x; q < H; q += NT) {
    const int k = perm_logical(q, H);
    s.g.xs[q] = f2bf(bfr(bf2f(w[k]) * bfr(s.g.xf[k] * r)));
  }
  __syncthreads();
}

// a bf16-valued fp32 vector of length K (global, shared between workgroups) -> lane-permuted bf16 at dst
__device__ __forceinline__ void load_vec_perm(const float* src, int K, uint16_t* dst) {
  for (int q = threadIdx.x; q < K; q += NT) dst[q] = f2bf(ld_ag(src + perm_logical(q, K)));
}

// ---------------------------------------------------------------- streaming GEMV
template <int K>
struct KS {
  static_assert(K % 64 == 0, "row length must be a multiple of 64");
  static constexpr int KB = K / 512;
  static constexpr int TM = (K % 512) / 64;      // stored elements per lane in the tail block
  static_assert(TM % 2 == 0, "tail block must give each lane whole dwords");
  static constexpr int TW = TM / 2;
};

template <int K>
struct RowRegs {
  u32x4 w[KS<K>::KB > 0 ? KS<K>::KB : 1];
  uint32_t t[KS<K>::TW > 0 ? KS<K>::TW : 1];
};

template <int K>
__device__ __forceinline__ void load_row(RowRegs<K>& r, const uint16_t* row, int lane) {
#pragma unroll
  for (int b = 0; b < KS<K>::KB; ++b) r.w[b] = __builtin_nontemporal_load((const u32x4*)(row + 512 * b + lane * 8));
#pragma unroll
  for (int t = 0; t < KS<K>::TW; ++t)
    r.t[t] = __builtin_nontemporal_load((const uint32_t*)(row + 512 * KS<K>::KB + lane * KS<K>::TM + 2 * t));
}

template <int K>
__device__ __forceinline__ float dot_row(const RowRegs<K>& r, const uint16_t* xs, int lane) {
  float acc = 0.0f;
#pragma unroll
  for (int b = 0; b < KS<K>::KB; ++b) {
    const u32x4 xv = *(const u32x4*)(xs + 512 * b + lane * 8);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc = __builtin_fmaf(bf_lo(r.w[b][j]), bf_lo(xv[j]), acc);
      acc = __builtin_fmaf(bf_hi(r.w[b][j]), bf_hi(xv[j]), acc);
    }
  }
#pragma unroll
  for (int t = 0; t < KS<K>::TW; ++t) {
    const uint32_t xv = *(const uint32_t*)(xs + 512 * KS<K>::KB + lane * KS<K>::TM + 2 * t);
    acc = __builtin_fmaf(bf_lo(r.t[t]), bf_lo(xv), acc);
    acc = __builtin_fmaf(bf_hi(r.t[t]), bf_hi(xv), acc);
  }
  return wave_sum_xor(acc);
}

// Long rows (more than 16 blocks of 512): streamed in segments of 8 blocks, the next segment's loads in flight
// while the current one is accumulated; the accumulation order is the same as dot_row's.
template <int K>
__device__ __forceinline__ float dot_row_long(const uint16_t* row, const uint16_t* xs, int lane) {
  constexpr int SEG = 8, NS = KS<K>::KB / SEG;
  static_assert(KS<K>::KB % SEG == 0 && KS<K>::TW == 0, "long rows are whole segments");
  u32x4 A[SEG], B[SEG];
  float acc = 0.0f;
  auto ld = [&](u32x4(&R)[SEG], int sg) {
#pragma unroll
    for (int b = 0; b < SEG; ++b) R[b] = __builtin_nontemporal_load((const u32x4*)(row + 512 * (sg * SEG + b) + lane * 8));
  };
  auto acc_seg = [&](const u32x4(&R)[SEG], int sg) {
#pragma unroll
    for (int b = 0; b < SEG; ++b) {
      const u32x4 xv = *(const u32x4*)(xs + 512 * (sg * SEG + b) + lane * 8);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc = __builtin_fmaf(bf_lo(R[b][j]), bf_lo(xv[j]), acc);
        acc = __builtin_fmaf(bf_hi(R[b][j]), bf_hi(xv[j]), acc);
      }
    }
  };
  ld(A, 0);
#pragma unroll 1
  for (int sg = 0; sg < NS; sg += 2) {
    if (sg + 1 < NS) ld(B, sg + 1);
    acc_seg(A, sg);
    if (sg + 2 < NS) ld(A, sg + 2);
    if (sg + 1 < NS) acc_seg(B, sg + 1);
  }
  return wave_sum_xor(acc);
}

// Groups of NR rows are dealt round-robin to the grid's waves; a wave streams its groups with the next
// group's loads in flight while it reduces the current one.  rowf(g, i) gives row i of group g (nullptr when
// absent), xf(i) its LDS input vector, epi(g, v) consumes the NR dot products (every lane holds them).
template <int K, int NR, class RowF, class XF, class EpiF>
__device__ __forceinline__ void gemv_run(int ngroups, int gw, int nw, RowF rowf, XF xf, EpiF epi) {
  const int lane = lane_id();
  int g = gw;
  if (g >= ngroups) return;
  if constexpr (KS<K>::KB > 16) {
    for (; g < ngroups; g += nw) {
      float v[NR];
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        const uint16_t* rp = rowf(g, i);
        v[i] = rp ? dot_row_long<K>(rp, xf(i), lane) : 0.0f;
      }
      epi(g, v);
    }
    return;
  }
  constexpr bool DB = NR * (KS<K>::KB + KS<K>::TW) <= 16;
  RowRegs<K> A[NR];
  auto load = [&](RowRegs<K>(&R)[NR], int gg) {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const uint16_t* rp = rowf(gg, i);
      if (rp) load_row<K>(R[i], rp, lane);
    }
  };
  auto comp = [&](RowRegs<K>(&R)[NR], int gg) {
    float v[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) v[i] = rowf(gg, i) ? dot_row<K>(R[i], xf(i), lane) : 0.0f;
    epi(gg, v);
  };
  load(A, g);
  if constexpr (DB) {
    RowRegs<K> B[NR];
    for (;;) {
      const int g2 = g + nw;
      if (g2 < ngroups) load(B, g2);
      comp(A, g);
      if (g2 >= ngroups) break;
      const int g3 = g2 + nw;
      if (g3 < ngroups) load(A, g3);
      comp(B, g2);
      if (g3 >= ngroups) break;
      g = g3;
    }
  } else {
    for (;;) {
      comp(A, g);
      g += nw;
      if (g >= ngroups) break;
      load(A, g);
    }
  }
}

// store NR values: lane i stores value i
template <int NR, class F>
__device__ __forceinline__ void lane_store(const float (&v)[NR], F f) {
  const int lane = lane_id();
#pragma unroll
  for (int i = 0; i < NR; ++i)
    if (lane == i) f(i, v[i]);
}

template <int V>
struct KC {
  static constexpr int value = V;
};

// run f with the compile-time row length equal to K (one of Ks...); other lengths are rejected by the host
template <int... Ks, class F>
__device__ __forceinline__ void dispatch_k(int K, F&& f) {
  (void)((K == Ks ? (f(KC<Ks>{}), true) : false) || ...);
}
#define MK_K_HIDDEN 256, 512, 1024, 2048, 4096
#define MK_K_ATTN 512, 1024, 2048, 4096
#define MK_K_MOE 256, 768
#define MK_K_INTER 1024, 12288

// ---------------------------------------------------------------- phases
// the step's input token; an id outside the vocabulary (only possible from corrupted state) reads row 0
__device__ __forceinline__ int token_of(const Params& p) {
  const int t = ld_ag_i(p.tokens + p.pos);
  return (t >= 0 && t < p.V) ? t : 0;
}

// P1: input RMSNorm + fused QKV GEMV (ref_numpy.py:111-115)
__device__ __forceinline__ void phase_qkv(const Params& p, int layer, Smem& s) {
  const LayerW& Lw = p.layers[layer];
  const bool first = layer == p.l0 && p.do_embed;
  const uint16_t* xrow = first ? p.embed + (size_t)token_of(p) * p.H : nullptr;
  build_norm_x(p, p.x, xrow, Lw.ln1, s);
  if (blockIdx.x == 0) {
    if (p.dump_x && layer > p.l0)
      for (int i = threadIdx.x; i < p.H; i += NT) p.dump_x[(size_t)(layer - 1) * p.H + i] = s.g.xf[i];
    if (layer == p.l0 && p.do_head && threadIdx.x == 0)
      __hip_atomic_store(p.amax, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const int rows = (p.NH + 2 * p.NKV) * p.HD;
  const int gw = blockIdx.x * NWAVE + wave_id(), nw = p.nwg * NWAVE;
  float* qkv = p.qkv;
  const uint16_t* W = Lw.wqkv;
  dispatch_k<MK_K_HIDDEN>(p.H, [&](auto kc_) {
    constexpr int KK = decltype(kc_)::value;
    gemv_run<KK, 2>(
      (rows + 1) / 2, gw, nw,
      [&](int g, int i) -> const uint16_t* { const int r = 2 * g + i; return r < rows ? W + (size_t)r * KK : nullptr; },
      [&](int) { return (const uint16_t*)s.g.xs; },
      [&](int g, const float(&v)[2]) {
        lane_store<2>(v, [&](int i, float val) { const int r = 2 * g + i; if (r < rows) st_ag(qkv + r, bfr(val)); });
      });
  });
}

// P2: per q head: q/k RMSNorm, neox RoPE, paged KV append, chunked softmax attention (ref_numpy.py:116-129)
__device__ __forceinline__ void phase_attn(const Params& p, int layer, Smem& s) {
  const int NKV = p.NKV, NH = p.NH, G = NH / NKV, HD = HDIM, BS = p.BS;
  // the G q heads of kv head g run on workgroups g%8 + 8*(j + G*(g/8)): one XCD per kv head
  const int wg = blockIdx.x;
  const int glo = wg & 7, t8 = wg >> 3, j = t8 % G, ghi = t8 / G, g = ghi * 8 + glo;
  if (g >= NKV || ghi * 8 + 8 > ((NKV + 7) & ~7)) return;
  const int h = g * G + j;
  const LayerW& Lw = p.layers[layer];
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  if (tid < HD) {
    s.a.q[tid] = ld_ag(p.qkv + (size_t)h * HD + tid);
    s.a.k[tid] = ld_ag(p.qkv + (size_t)(NH + g) * HD + tid);
    s.a.v[tid] = ld_ag(p.qkv + (size_t)(NH + NKV + g) * HD + tid);
  }
  __syncthreads();
  if (wave < 2) {
    float* vec = wave == 0 ? s.a.q : s.a.k;
    float a0 = vec[lane], a1 = vec[lane + 64];
    if (p.qk_norm) {                                   // ref_numpy.py:116-118, per-head RMSNorm
      const uint16_t* w = wave == 0 ? Lw.qn : Lw.kn;
      float acc = __builtin_fmaf(a0, a0, 0.0f);
      acc = __builtin_fmaf(a1, a1, acc);
      acc = wave_sum_xor(acc);
      const float r = 1.0f / __builtin_sqrtf(acc / (float)HD + p.eps);
      a0 = bfr(bf2f(w[lane]) * bfr(a0 * r));
      a1 = bfr(bf2f(w[lane + 64]) * bfr(a1 * r));
    }
    const float c = p.rope_cos[(size_t)p.pos * (HD / 2) + lane];   // ref_numpy.py:84-88 rotate_half
    const float sn = p.rope_sin[(size_t)p.pos * (HD / 2) + lane];
    vec[lane] = bfr(bfr(a0 * c) + bfr(-a1 * sn));
    vec[lane + 64] = bfr(bfr(a1 * c) + bfr(a0 * sn));
  }
  __syncthreads();
  const int pos = p.pos, n = pos + 1, nch = (n + CHUNK - 1) / CHUNK;
  {                                                     // paged append: K [blk][NKV][HD/8][BS][8], V [blk][NKV][HD][BS]
    const int blk = p.btab[pos / BS], off = pos % BS;
    if (j == 0 && tid < HD) {
      Lw.kc[((((size_t)blk * NKV + g) * (HD / 8) + tid / 8) * BS + off) * 8 + tid % 8] = f2bf(s.a.k[tid]);
      Lw.vc[(((size_t)blk * NKV + g) * HD + tid) * BS + off] = f2bf(s.a.v[tid]);
    }
  }
  // scores: lane = position inside a chunk; s_t = (q . k_t in ascending d) * scale
  for (int c = wave; c < nch; c += NWAVE) {
    const int t = c * CHUNK + lane;
    float sc = -__builtin_huge_valf();
    if (t < n) {
      float acc = 0.0f;
      if (t == pos) {
#pragma unroll 16
        for (int d = 0; d < HD; ++d) acc = __builtin_fmaf(s.a.q[d], s.a.k[d], acc);
      } else {
        const int blk = p.btab[t / BS], off = t % BS;
        const uint16_t* kp = Lw.kc + (((size_t)blk * NKV + g) * (HD / 8)) * BS * 8 + off * 8;
#pragma unroll 4
        for (int jj = 0; jj < HD / 8; ++jj) {
          const u32x4 kv = *(const u32x4*)(kp + (size_t)jj * BS * 8);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            acc = __builtin_fmaf(s.a.q[8 * jj + 2 * e], bf_lo(kv[e]), acc);
            acc = __builtin_fmaf(s.a.q[8 * jj + 2 * e + 1], bf_hi(kv[e]), acc);
          }
        }
      }
      sc = acc * p.attn_scale;
    }
    const float m = wave_max(sc);
    if (t < n) s.a.p[t] = expf_mk(sc - m);
    if (lane == 0) s.a.mc[c] = m;
  }
  __syncthreads();
  // per chunk and dim: a_c[d] = sum_t p_t v_t[d] (ascending t), l_c = sum_t p_t
  for (int item = tid; item < nch * HD; item += NT) {
    const int c = item / HD, d = item % HD;
    const int t0 = c * CHUNK, t1 = min(t0 + CHUNK, n);
    float a = 0.0f, l = 0.0f;
    for (int tb = t0; tb < t1; tb += BS) {
      const int blk = p.btab[tb / BS];
      const uint16_t* vp = Lw.vc + (((size_t)blk * NKV + g) * HD + d) * BS;
      const u32x4 va = *(const u32x4*)vp;
      const u32x4 vb = *(const u32x4*)(vp + 8);
      const int te = min(tb + BS, t1) - tb;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (i < te) {
          const uint32_t wv = i < 8 ? va[i >> 1] : vb[(i - 8) >> 1];
          const float vb16 = (i & 1) ? bf_hi(wv) : bf_lo(wv);
          const int t = tb + i;
          const float pt = s.a.p[t];
          a = __builtin_fmaf(pt, t == pos ? s.a.v[d] : vb16, a);
          l = l + pt;
        }
      }
    }
    s.a.ac[c][d] = a;
    if (d == 0) s.a.lc[c] = l;
  }
  __syncthreads();
  if (tid < HD) {                                       // merge chunks in ascending order
    float M = -__builtin_huge_valf();
    for (int c = 0; c < nch; ++c) M = fmaxf(M, s.a.mc[c]);
    float Ls = 0.0f, A = 0.0f;
    for (int c = 0; c < nch; ++c) {
      const float w = expf_mk(s.a.mc[c] - M);
      Ls = __builtin_fmaf(w, s.a.lc[c], Ls);
      A = __builtin_fmaf(w, s.a.ac[c][tid], A);
    }
    st_ag(p.o + (size_t)h * HD + tid, bfr(A / Ls));
  }
}

// P3: O projection and residual (ref_numpy.py:130): x = bfr(x + bfr(Wo . o))
__device__ __forceinline__ void phase_oproj(const Params& p, int layer, Smem& s) {
  const LayerW& Lw = p.layers[layer];
  const int K = p.NH * p.HD, H = p.H;
  load_vec_perm(p.o, K, s.g.xs);
  __syncthreads();
  const bool first = layer == p.l0 && p.do_embed;
  const uint16_t* xrow = first ? p.embed + (size_t)token_of(p) * H : nullptr;
  const int gw = blockIdx.x * NWAVE + wave_id(), nw = p.nwg * NWAVE;
  float* x = p.x;
  const uint16_t* W = Lw.wo;
  dispatch_k<MK_K_ATTN>(K, [&](auto kc_) {
    constexpr int KK = decltype(kc_)::value;
    gemv_run<KK, 2>(
      (H + 1) / 2, gw, nw,
      [&](int g, int i) -> const uint16_t* { const int r = 2 * g + i; return r < H ? W + (size_t)r * KK : nullptr; },
      [&](int) { return (const uint16_t*)s.g.xs; },
      [&](int g, const float(&v)[2]) {
        lane_store<2>(v, [&](int i, float val) {
          const int r = 2 * g + i;
          if (r < H) {
            const float xo = xrow ? bf2f(xrow[r]) : ld_ag(x + r);
            st_ag(x + r, bfr(xo + bfr(val)));
          }
        });
      });
  });
}

// P4: post-attention RMSNorm + router GEMV (ref_numpy.py:131-134)
__device__ __forceinline__ void phase_router(const Params& p, int layer, Smem& s) {
  const LayerW& Lw = p.layers[layer];
  build_norm_x(p, p.x, nullptr, Lw.ln2, s);
  const int E = p.E;
  const int gw = blockIdx.x * NWAVE + wave_id(), nw = p.nwg * NWAVE;
  float* lg = p.logits;
  const uint16_t* W = Lw.wr;
  dispatch_k<MK_K_HIDDEN>(p.H, [&](auto kc_) {
    constexpr int KK = decltype(kc_)::value;
    gemv_run<KK, 2>(
      (E + 1) / 2, gw, nw,
      [&](int g, int i) -> const uint16_t* { const int r = 2 * g + i; return r < E ? W + (size_t)r * KK : nullptr; },
      [&](int) { return (const uint16_t*)s.g.xs; },
      [&](int g, const float(&v)[2]) {
        lane_store<2>(v, [&](int i, float val) { const int r = 2 * g + i; if (r < E) st_ag(lg + r, bfr(val)); });
      });
  });
}

// softmax top-k over the router logits (ref_numpy.py:135-140) into s.ids / s.wts / s.order (wave 0 computes;
// every workgroup recomputes it, so no phase is spent on it).
__device__ __forceinline__ void route_topk(const Params& p, Smem& s) {
  const int E = p.E, K = p.TOPK;
  if (wave_id() == 0) {
    const int lane = lane_id();
    float m = -__builtin_huge_valf();
    for (int e = lane; e < E; e += 64) {
      const float v = ld_ag(p.logits + e);
      s.prob[e] = v;
      m = fmaxf(m, v);
    }
    m = wave_max(m);
    float acc = 0.0f;
    for (int e = lane; e < E; e += 64) {
      const float ex = expf_mk(s.prob[e] - m);
      s.prob[e] = ex;
      acc = acc + ex;
    }
    const float S = wave_sum_xor(acc);
    for (int e = lane; e < E; e += 64) s.prob[e] = s.prob[e] / S;
    // K rounds of (max probability, lowest id); lane l owns experts l, l+64, l+128, l+192
    float sel = 0.0f;
    bool taken[MAX_E / 64] = {false, false, false, false};
    for (int k = 0; k < K; ++k) {
      float bv = -1.0f;
      int bi = 0x7fffffff;
#pragma unroll
      for (int w = 0; w < MAX_E / 64; ++w) {
        const int e = lane + 64 * w;
        if (e < E && !taken[w]) {
          const float v = s.prob[e];
          if (v > bv) { bv = v; bi = e; }
        }
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
#pragma unroll
      for (int w = 0; w < MAX_E / 64; ++w)
        if (lane + 64 * w == bi) taken[w] = true;
      if (bi >= E) bi = 0;                               // non-finite probabilities: keep the index in range
      if (lane == 0) { s.ids[k] = bi; s.wts[k] = bv; }
      sel = sel + bv;
    }
    if (lane == 0) {
      for (int k = 0; k < K; ++k) s.wts[k] = bfr(p.norm_topk ? s.wts[k] / sel : s.wts[k]);
      for (int k = 0; k < K; ++k) s.order[k] = k;          // slots in ascending expert id (index_add_ order)
      for (int a = 1; a < K; ++a)
        for (int b = a; b > 0 && s.ids[s.order[b]] < s.ids[s.order[b - 1]]; --b) {
          const int t = s.order[b]; s.order[b] = s.order[b - 1]; s.order[b - 1] = t;
        }
    }
  }
  __syncthreads();
}

// P5: experts gate/up + SiLU*up for the top-k slots (ref_numpy.py:142-145)
__device__ __forceinline__ void phase_expert_up(const Params& p, int layer, Smem& s) {
  const LayerW& Lw = p.layers[layer];
  route_topk(p, s);
  if (blockIdx.x == 0 && threadIdx.x < 64) {
    const int t = threadIdx.x;
    if (p.dump_ids && t < p.TOPK) p.dump_ids[(size_t)layer * p.TOPK + t] = s.ids[t];
    if (p.dump_wts && t < p.TOPK) p.dump_wts[(size_t)layer * p.TOPK + t] = s.wts[t];
    if (p.dump_logits)
      for (int e = t; e < p.E; e += 64) p.dump_logits[(size_t)layer * p.E + e] = ld_ag(p.logits + e);
  }
  build_norm_x(p, p.x, nullptr, Lw.ln2, s);
  const int MI = p.MI, H = p.H, KT = p.TOPK;
  const int gw = blockIdx.x * NWAVE + wave_id(), nw = p.nwg * NWAVE;
  float* hb = p.hbuf;
  const uint16_t* W = Lw.w13;
  dispatch_k<MK_K_HIDDEN>(H, [&](auto kc_) {
    constexpr int KK = decltype(kc_)::value;
    gemv_run<KK, 2>(
      KT * MI, gw, nw,
      [&](int g, int i) -> const uint16_t* {
        const int slot = g / MI, jj = g - slot * MI;
        return W + ((size_t)s.ids[slot] * 2 * MI + 2 * jj + i) * KK;
      },
      [&](int) { return (const uint16_t*)s.g.xs; },
      [&](int g, const float(&v)[2]) {
        if (lane_id() == 0) st_ag(hb + g, bfr(bfr(silu(bfr(v[0]))) * bfr(v[1])));
      });
  });
}

// P6: expert down, routing weight, combine in ascending expert id, residual (ref_numpy.py:146-148)
__device__ __forceinline__ void phase_expert_down(const Params& p, int layer, Smem& s) {
  const LayerW& Lw = p.layers[layer];
  route_topk(p, s);
  const int MI = p.MI, H = p.H, KT = p.TOPK;
  for (int slot = 0; slot < KT; ++slot) load_vec_perm(p.hbuf + (size_t)slot * MI, MI, s.g.xs + (size_t)slot * MI);
  __syncthreads();
  const int gw = blockIdx.x * NWAVE + wave_id(), nw = p.nwg * NWAVE;
  float* x = p.x;
  const uint16_t* W = Lw.w2;
  dispatch_k<MK_K_MOE>(MI, [&](auto kc_) {
    constexpr int KK = decltype(kc_)::value;
    gemv_run<KK, MAX_TOPK>(
      H, gw, nw,
      [&](int g, int i) -> const uint16_t* { return i < KT ? W + ((size_t)s.ids[i] * H + g) * KK : nullptr; },
      [&](int i) { return (const uint16_t*)(s.g.xs + (size_t)i * KK); },
      [&](int g, const float(&v)[MAX_TOPK]) {
        if (lane_id() == 0) {
          float y[MAX_TOPK];
#pragma unroll
          for (int i = 0; i < MAX_TOPK; ++i) y[i] = i < KT ? bfr(bfr(v[i]) * s.wts[i]) : 0.0f;
          float acc = 0.0f;
          for (int k = 0; k < KT; ++k) {
            const int o = s.order[k];
            float yk = 0.0f;
#pragma unroll
            for (int i = 0; i < MAX_TOPK; ++i) yk = (o == i) ? y[i] : yk;
            acc = bfr(acc + yk);
          }
          st_ag(x + g, bfr(ld_ag(x + g) + acc));
        }
      });
  });
}

// dense MLP (ref_numpy.py:149-152): P4' gate/up + SiLU*up, P5' down + residual
__device__ __forceinline__ void phase_gateup(const Params& p, int layer, Smem& s) {
  const LayerW& Lw = p.layers[layer];
  build_norm_x(p, p.x, nullptr, Lw.ln2, s);
  const int I = p.I;
  const int gw = blockIdx.x * NWAVE + wave_id(), nw = p.nwg * NWAVE;
  float* hb = p.hbuf;
  const uint16_t* W = Lw.wgu;
  dispatch_k<MK_K_HIDDEN>(p.H, [&](auto kc_) {
    constexpr int KK = decltype(kc_)::value;
    gemv_run<KK, 2>(
      I, gw, nw,
      [&](int g, int i) -> const uint16_t* { return W + ((size_t)2 * g + i) * KK; },
      [&](int) { return (const uint16_t*)s.g.xs; },
      [&](int g, const float(&v)[2]) {
        if (lane_id() == 0) st_ag(hb + g, bfr(bfr(silu(bfr(v[0]))) * bfr(v[1])));
      });
  });
}

__device__ __forceinline__ void phase_down(const Params& p, int layer, Smem& s) {
  const LayerW& Lw = p.layers[layer];
  const int I = p.I, H = p.H;
  load_vec_perm(p.hbuf, I, s.g.xs);
  __syncthreads();
  const int gw = blockIdx.x * NWAVE + wave_id(), nw = p.nwg * NWAVE;
  float* x = p.x;
  const uint16_t* W = Lw.wd;
  dispatch_k<MK_K_INTER>(I, [&](auto kc_) {
    constexpr int KK = decltype(kc_)::value;
    gemv_run<KK, 1>(
      H, gw, nw,
      [&](int g, int) -> const uint16_t* { return W + (size_t)g * KK; },
      [&](int) { return (const uint16_t*)s.g.xs; },
      [&](int g, const float(&v)[1]) {
        if (lane_id() == 0) st_ag(x + g, bfr(ld_ag(x + g) + bfr(v[0])));
      });
  });
}

// P7: final norm + lm_head + per-wave argmax folded into one 64-bit key (ref_numpy.py:155-158; first maximum wins)
__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {
  if (v == 0.0f) v = 0.0f;                                // -0 and +0 compare equal, as in torch.argmax
  const uint32_t u = f2bits(v);
  const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)idx);
}

__device__ __forceinline__ void phase_head(const Params& p, Smem& s) {
  build_norm_x(p, p.x, nullptr, p.final_norm, s);
  if (blockIdx.x == 0 && p.dump_x)
    for (int i = threadIdx.x; i < p.H; i += NT) p.dump_x[(size_t)(p.l1 - 1) * p.H + i] = s.g.xf[i];
  const int V = p.V;
  const int gw = blockIdx.x * NWAVE + wave_id(), nw = p.nwg * NWAVE;
  const uint16_t* W = p.lm_head;
  uint64_t best = 0;
  dispatch_k<MK_K_HIDDEN>(p.H, [&](auto kc_) {
    constexpr int KK = decltype(kc_)::value;
    gemv_run<KK, 2>(
      (V + 1) / 2, gw, nw,
      [&](int g, int i) -> const uint16_t* { const int r = 2 * g + i; return r < V ? W + (size_t)r * KK : nullptr; },
      [&](int) { return (const uint16_t*)s.g.xs; },
      [&](int g, const float(&v)[2]) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int r = 2 * g + i;
          if (r < V) {
            const uint64_t key = argmax_key(bfr(v[i]), r);
            best = key > best ? key : best;
          }
        }
      });
  });
  if (lane_id() == 0 && best) __hip_atomic_fetch_max(p.amax, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void phase_token(const Params& p) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const uint64_t key = ld_ag64(p.amax);
    int32_t tok = (int32_t)(0xFFFFFFFFu - (uint32_t)key);
    if (key == 0 || tok < 0 || tok >= p.V) {              // no finite logit was seen: flag it, keep the id valid
      st_ag_i(p.abort_word, 3);
      tok = 0;
    }
    st_ag_i(p.out_tokens + p.pos, tok);
    if (p.write_next) st_ag_i(p.tokens + p.pos + 1, tok);
  }
}

// ---------------------------------------------------------------- kernels
enum Phase { PH_QKV = 0, PH_ATTN, PH_OPROJ, PH_ROUTER, PH_EXPUP, PH_EXPDN, PH_GATEUP, PH_DOWN, PH_HEAD, PH_TOKEN };

__device__ __forceinline__ void run_phase(const Params& p, int ph, int layer, Smem& s) {
  switch (ph) {
    case PH_QKV: phase_qkv(p, layer, s); break;
    case PH_ATTN: phase_attn(p, layer, s); break;
    case PH_OPROJ: phase_oproj(p, layer, s); break;
    case PH_ROUTER: phase_router(p, layer, s); break;
    case PH_EXPUP: phase_expert_up(p, layer, s); break;
    case PH_EXPDN: phase_expert_down(p, layer, s); break;
    case PH_GATEUP: phase_gateup(p, layer, s); break;
    case PH_DOWN: phase_down(p, layer, s); break;
    case PH_HEAD: phase_head(p, s); break;
    case PH_TOKEN: phase_token(p); break;
  }
}

extern "C" __global__ void __launch_bounds__(NT, 1) etxmk_fused(Params p) {
  __shared__ Smem s;
  int k = 0;
  for (int layer = p.l0; layer < p.l1; ++layer) {
    phase_qkv(p, layer, s);
    if (!grid_sync(p, k, s)) return;
    phase_attn(p, layer, s);
    if (!grid_sync(p, k, s)) return;
    phase_oproj(p, layer, s);
    if (!grid_sync(p, k, s)) return;
    if (p.moe) {
      phase_router(p, layer, s);
      if (!grid_sync(p, k, s)) return;
      phase_expert_up(p, layer, s);
      if (!grid_sync(p, k, s)) return;
      phase_expert_down(p, layer, s);
      if (!grid_sync(p, k, s)) return;
    } else {
      phase_gateup(p, layer, s);
      if (!grid_sync(p, k, s)) return;
      phase_down(p, layer, s);
      if (!grid_sync(p, k, s)) return;
    }
  }
  if (p.do_head) {
    phase_head(p, s);
    if (!grid_sync(p, k, s)) return;
    phase_token(p);
  }
}

// unfused mode: one kernel per phase, same device functions (named per phase so profiles separate them)
#define MK_PHASE_KERNEL(name, PH)                                               \
  extern "C" __global__ void __launch_bounds__(NT, 1) name(Params p, int layer) { \
    __shared__ Smem s;                                                          \
    run_phase(p, PH, layer, s);                                                 \
  }
MK_PHASE_KERNEL(etxmk_p_qkv, PH_QKV)
MK_PHASE_KERNEL(etxmk_p_attn, PH_ATTN)
MK_PHASE_KERNEL(etxmk_p_oproj, PH_OPROJ)
MK_PHASE_KERNEL(etxmk_p_router, PH_ROUTER)
MK_PHASE_KERNEL(etxmk_p_expert_up, PH_EXPUP)
MK_PHASE_KERNEL(etxmk_p_expert_down, PH_EXPDN)
MK_PHASE_KERNEL(etxmk_p_gateup, PH_GATEUP)
MK_PHASE_KERNEL(etxmk_p_down, PH_DOWN)
MK_PHASE_KERNEL(etxmk_p_head, PH_HEAD)
MK_PHASE_KERNEL(etxmk_p_token, PH_TOKEN)

// ---------------------------------------------------------------- seeded initialisation / packing
// n_t consecutive tensors of rows x cols (experts of one layer); element (r, k) of tensor e is number r*cols+k
// of stream sid0 + e; stored at its lane-permuted position when perm != 0.
extern "C" __global__ void etxmk_gen_weights(uint16_t* dst, uint64_t seed, uint64_t sid0, int n_t, int rows, int cols,
                                             int perm, float scale) {
  const size_t per = (size_t)rows * cols;
  const size_t total8 = per * n_t / 8;
  for (size_t q8 = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q8 < total8; q8 += (size_t)gridDim.x * blockDim.x) {
    const size_t q = q8 * 8;
    const int e = (int)(q / per);
    const size_t rem = q - (size_t)e * per;
    const int r = (int)(rem / cols), p0 = (int)(rem - (size_t)r * cols);
    const uint64_t key = stream_key(seed, sid0 + (uint64_t)e);
    uint16_t out[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = perm ? perm_logical(p0 + u, cols) : p0 + u;
      out[u] = f2bf(scale * normal_at(key, (uint64_t)r * cols + k));
    }
    *(u32x4*)(dst + q) = *(const u32x4*)out;
  }
}

extern "C" __global__ void etxmk_fill_u16(uint16_t* dst, size_t n, uint16_t v) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) dst[i] = v;
}

extern "C" __global__ void etxmk_pack_rows(uint16_t* dst, const uint16_t* src, int rows, int cols) {
  const size_t total = (size_t)rows * cols;
  for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total; q += (size_t)gridDim.x * blockDim.x) {
    const int r = (int)(q / cols), p = (int)(q - (size_t)r * cols);
    dst[q] = src[(size_t)r * cols + perm_logical(p, cols)];
  }
}

// KV positions [0, npos): element (t, h, d) is number (t*NKV + h)*HD + d of the layer's K / V stream
extern "C" __global__ void etxmk_gen_kv(uint16_t* kc, uint16_t* vc, const int32_t* btab, uint64_t kkey, uint64_t vkey,
                                        int npos, int NKV, int HD, int BS) {
  const size_t total = (size_t)npos * NKV * HD;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int d = (int)(i % HD), h = (int)((i / HD) % NKV), t = (int)(i / ((size_t)HD * NKV));
    const int blk = btab[t / BS], off = t % BS;
    kc[((((size_t)blk * NKV + h) * (HD / 8) + d / 8) * BS + off) * 8 + d % 8] = f2bf(normal_at(kkey, i));
    vc[(((size_t)blk * NKV + h) * HD + d) * BS + off] = f2bf(normal_at(vkey, i));
  }
}

}  // namespace mk
