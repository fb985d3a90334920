#pragma once
// DeepSeek-V2 decode step (multi-head latent attention, shared experts, dense leading layers) as one persistent
// launch for up to 4 sequences, built on the batched kernel's machinery (mk_batch.h): a batch equals one step per
// sequence bit for bit, and a single sequence runs as a batch of one.
//
// Reference path: examples/dsv2lite/results/2026-10-14-k1/b_alld4r0l1kvs_stamps/fleet_src/host/reference_decode.py
// (the numerical specification of the reference's DeepSeek-V2-Lite host, kept as a snapshot): :78-118 yarn RoPE
// tables, :120-136 RoPE, :198-206 softmax scale, :210-256 absorbed attention, :259-291 MLP and MoE, :294-302 layer.
//
// Phases of a layer:
//   P1  input RMSNorm + GEMV over the fused [q_proj; kv_a_proj_with_mqa] rows          -> qkv [B][NQA] (bf16 values)
//   P1b absorbed queries q_c[h] = W_UK[h]^T q_nope[h] (fp32, not rounded)                -> qc (one buffer per layer)
//   P2  latent attention per (sequence, head group of 8, 64-position chunk): the chunk holding the current position
//       builds the new latent row (kv_a_layernorm, RoPE of k_pe) and appends it to the cache; s = (q_c . c +
//       q_pe . k_pe) * scale, chunk softmax partials (a, m, l)                               -> apart
//   P2c per (sequence, head, quarter of v_head): merge of the partials into o_c (fp32), then
//       out[h*v_head + d] = bfr(W_UV[h][d] . o_c[h])                                     -> o16
//   P3  O projection + residual (mk_batch.h)
//   MoE layers: P4 post-attention RMSNorm, fp32 router logits and the shared experts' gate/up | P5 top-k with fp32
//   weights (probability * routed_scale) and the routed gate/up | P6 routed and shared down, combine, residual
//   dense layers: gate/up | down, rows padded to the row format (the pads are zero weights and zero inputs)
// Latent cache: [block][(kv_lora + qk_rope) / 8][block_size][8] bf16, the Qwen3 K layout with one kv head of 576.
#include "mk_batch.h"

namespace mk {

constexpr int MLA_KVL = 512;              // kv_lora_rank
constexpr int MLA_NOPE = 128;             // qk_nope_head_dim
constexpr int MLA_R = 64;                 // qk_rope_head_dim
constexpr int MLA_VH = 128;               // v_head_dim
constexpr int MLA_QD = MLA_NOPE + MLA_R;  // q head dim
constexpr int MLA_CD = MLA_KVL + MLA_R;   // latent cache row
constexpr int MLA_CG = MLA_CD / 8;        // 16-byte dim groups of a latent row
constexpr int MLA_G = 8;                  // heads per attention item
constexpr int MLA_PART = MLA_KVL + 2;     // attention partial: a[kv_lora], m, l
constexpr int MLA_MAX_NH = 32;
constexpr int MAX_B_DS = 4;             // sequences per DeepSeek-V2 step

// LDS of the attention phase.  Tile slot [j][u] holds dims 8j..8j+7 of chunk position u ^ (j & 15): a lane reading
// position t of group j (scores: lane = position) and a lane reading group j of position t (P.V: lane = group)
// both touch 64 distinct 16-byte slots whose bank groups differ within every 16 lanes.
struct MlaTiles {
  u32x4 t[MLA_CG][CHUNK];
  alignas(16) float xo[MLA_KVL];          // P2c: o_c of the item, in the W_UV rows' stored order
  alignas(16) float p[MLA_G][2 * MAX_CHUNKS];  // chunk: exp(s - m) per position; merge: chunk weights, chunk sums
  float m[MLA_G];
};

template <int B, int XC>
struct SmemD {
  static constexpr int NCAP = B * MAX_H > 32768 ? 32768 : B * MAX_H;
  static constexpr bool NORM_HOIST = false;             // per-row weight loads in build_norm_xb (registers)
  static constexpr int XCAP = XC;
  union {
    struct {
      alignas(16) uint16_t xr[NCAP];
      alignas(16) uint16_t xs[NCAP];
    } n;
    struct {
      alignas(16) uint16_t xs[XCAP];
      float xres[B][RES_ROWS];
      float acc[B][RES_ROWS];
      float sh[B][RES_ROWS];              // shared experts' down projection of this workgroup's output rows
    } v;
    MlaTiles a;
  };
  float rs[B];
  int32_t rids[B][MAX_TOPK];
  float rwts[B][MAX_TOPK];
  int32_t pexp[MAX_PAIRS];
  int32_t pseq[MAX_PAIRS];
  float pw[MAX_PAIRS];
  int32_t uexp[MAX_PAIRS];
  int32_t ustart[MAX_PAIRS + 1];
  int32_t nexp;
  int32_t bpair[B][MAX_TOPK];           // route_all's per-sequence pair lists (unused by these kernels)
  uint32_t kbits[KEY_WORDS];
  uint32_t kpre[KEY_WORDS];
  int32_t abort, last, phase;
};

__device__ __forceinline__ void st_ag2(float* p, float a, float b) {
  const uint64_t v = (uint64_t)f2bits(a) | ((uint64_t)f2bits(b) << 32);
  __hip_atomic_store((MK_G uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ld_ag2(const float* p, float& a, float& b) {
  const uint64_t v = ld_ag64((const uint64_t*)p);
  a = bits2f((uint32_t)v);
  b = bits2f((uint32_t)(v >> 32));
}

// DeepSeek RoPE of the pair (x[2i], x[2i+1]) (reference_decode.py:120-136: de-interleave, then rotate_half):
// out[i] = x[2i] c - x[2i+1] s, out[i + 32] = x[2i+1] c + x[2i] s, each product and sum in fp32, then bf16
__device__ __forceinline__ void rope_ds_pair(float a, float b, float c, float s, float& lo, float& hi) {
  lo = bfr(a * c + (-b) * s);
  hi = bfr(b * c + a * s);
}

// The latent row of row b's QKV output at position q, one wave: c = kv_a_layernorm(kv_a) (reference_decode.py:231;
// the sum of squares in dot order, then bfr(w * bfr(x * r))) and k_pe roped at q (:234), as fp32 (bf16 values) in
// registers: lane l holds c[l + 64e] in c[e], and lanes < 32 the roped pair (lo, hi) = dims 512 + l, 544 + l.
struct LatentRow {
  float c[MLA_KVL / 64];
  float lo, hi;
};
__device__ __forceinline__ LatentRow latent_row(const Params& p, const LayerW& Lw, int b, int q) {
  const int lane = lane_id();
  const float* kva = p.qkv + (size_t)b * p.nqkv + p.NH * MLA_QD;
  LatentRow r;
  float x[MLA_KVL / 64];
#pragma unroll
  for (int e = 0; e < MLA_KVL / 64; ++e) x[e] = ld_ag(kva + lane + 64 * e);
  float a0 = 0.0f, a1 = 0.0f;
  if (lane < MLA_R / 2) { a0 = ld_ag(kva + MLA_KVL + 2 * lane); a1 = ld_ag(kva + MLA_KVL + 2 * lane + 1); }
  float acc = 0.0f;
#pragma unroll
  for (int e = 0; e < MLA_KVL / 64; ++e) acc = __builtin_fmaf(x[e], x[e], acc);
  acc = wave_sum(acc);
  const float rs = 1.0f / __builtin_sqrtf(acc / (float)MLA_KVL + p.eps);
#pragma unroll
  for (int e = 0; e < MLA_KVL / 64; ++e) r.c[e] = bfr(bf2f(ld_u16(Lw.kn + lane + 64 * e)) * bfr(x[e] * rs));
  r.lo = r.hi = 0.0f;
  if (lane < MLA_R / 2) {
    const float cs = ld_f(p.rope_cos + (size_t)q * (MLA_R / 2) + lane);
    const float sn = ld_f(p.rope_sin + (size_t)q * (MLA_R / 2) + lane);
    rope_ds_pair(a0, a1, cs, sn, r.lo, r.hi);
  }
  return r;
}
// visit (dim, value) of a latent row held as above
template <class F>
__device__ __forceinline__ void latent_dims(const LatentRow& r, F f) {
  const int lane = lane_id();
#pragma unroll
  for (int e = 0; e < MLA_KVL / 64; ++e) f(lane + 64 * e, r.c[e]);
  if (lane < MLA_R / 2) {
    f(MLA_KVL + lane, r.lo);
    f(MLA_KVL + MLA_R / 2 + lane, r.hi);
  }
}

// the absorbed queries of (layer, sequence b, head h)
__device__ __forceinline__ float* qc_of(const Params& p, int layer, int b, int h) {
  return p.qc + (((size_t)layer * p.B + b) * p.NH + h) * MLA_KVL;
}

// P1b: q_c[b][h][i] = sum_d q_nope[b][h][d] * W_UK[h][d][i] (reference_decode.py:245-249), the canonical dot of
// the W_UK^T row (h, i) (qk_nope long) with the bf16 q_nope of (b, h), kept in fp32
template <int B, class S, class Wait>
__device__ __forceinline__ void phase_absorb_b(const Params& p, int layer, S& s, Wait wait) {
  using WR = Bf16Row<MLA_NOPE>;
  constexpr int NR = 4;
  static_assert(B * MLA_MAX_NH * MLA_NOPE <= S::XCAP, "query rows exceed the LDS budget");
  const LayerW Lw = layer_w(p, layer);
  const int NH = p.NH, nb = p.B, rows = NH * MLA_KVL, nqkv = p.nqkv;
  gemv_run_b<WR, NR, B>(
      rows / NR, [&](int g, int i) -> const uint8_t* { return mrow<WR>(Lw.wuk, (size_t)g * NR + i); },
      [&](int) { return nb; },
      [&](int g, int b) { return (const uint16_t*)(s.v.xs + (b * NH + (g * NR) / MLA_KVL) * MLA_NOPE); },
      [&](int g, int nv, const float(&v)[NR][B]) {
        lane_store_b<NR, B>(v, nv, [&](int i, int b, float val, bool ok) {
          st_ag(ok ? qc_of(p, layer, b, 0) + g * NR + i : sink_of(p), val);
        });
      },
      [&]() {
        if (!wait()) return false;
        constexpr int C8 = MLA_NOPE / 8;                  // q_nope of every (sequence, head), lane-permuted bf16
        for (int c = threadIdx.x; c < nb * NH * C8; c += NT) {
          const int vec = c / C8, q = 8 * (c - vec * C8), b = vec / NH, h = vec - b * NH;
          const float* src = p.qkv + (size_t)b * nqkv + h * MLA_QD;
          float v[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = ld_ag(src + perm_logical(q + e, MLA_NOPE));
          uint32_t o[4];
#pragma unroll
          for (int e = 0; e < 8; e += 2) o[e / 2] = (uint32_t)f2bf(v[e]) | ((uint32_t)f2bf(v[e + 1]) << 16);
          *(u32x4*)(s.v.xs + 8 * c) = u32x4{o[0], o[1], o[2], o[3]};
        }
        __syncthreads();
        return true;
      },
      p.nwg, p.trace, s.phase);
}

struct MlaItem {
  int b, hg, c, pos;
};
// items are numbered sequence by sequence (p.ibase), head group fastest
__device__ __forceinline__ MlaItem mla_item(const Params& p, int item, int NHG) {
  int b = 0;
  while (b + 1 < p.B && item >= p.ibase[b + 1]) ++b;
  const int r = item - p.ibase[b];
  return MlaItem{b, r % NHG, r / NHG, p.posb[b]};
}

// P2: absorbed attention over the latent cache (reference_decode.py:250-253 in chunked form).  Per item (sequence
// b, head group, chunk c of positions 0..pos): s_t = ((q_c . c_t over kv_lora, one ascending fma chain) +
// (q_pe . k_pe_t over qk_rope, ascending)) * scale; the chunk's max m, p_t = exp(s_t - m), l = sum p_t and
// a[i] = sum_t p_t c_t[i] (ascending t) -> the chunk partial (a, m, l).  The merge follows in P2c.
template <int B, class S, class Wait>
__device__ __forceinline__ void phase_mla_attn(const Params& p, int layer, S& s, Wait wait) {
  static_assert(MLA_G == NWAVE, "one head per wave");
  const int NH = p.NH, GH = NH < MLA_G ? NH : MLA_G, NHG = NH / GH, BS = p.BS;
  const int nitems = p.ibase[p.B];
  const LayerW Lw = layer_w(p, layer);
  const int lane = lane_id(), wave = wave_u();
  // the chunk's cached latent rows, HBM -> LDS (global_load_lds, 16 bytes per lane): wave w copies groups w, w+8, ...
  // (the rows do not depend on this step, so the first item's copies are issued before the wait; the current
  // position's row is computed here instead)
  // positions from first_new(pos) on are this launch's (the row's own, and in prefill the earlier rows'): built
  // from the rows' QKV outputs, not read from the cache
  auto first_new = [&](int pos) { return p.pf ? p.posb[0] : pos; };
  auto load_tile = [&](const MlaItem& it) {
    const int t0 = it.c * CHUNK, n = it.pos + 1, fp = first_new(it.pos);
    const int g16 = t0 + (lane & ~15);                   // the swizzle permutes inside 16 positions: one block
    const int blk = g16 < n ? ld_i(p.btab + (size_t)it.b * p.nbps + g16 / BS) : 0;
    for (int j = wave; j < MLA_CG; j += NWAVE) {
      const int T = t0 + (lane ^ (j & 15));
      if (T < n && T < fp)
        __builtin_amdgcn_global_load_lds((const MK_G void*)(Lw.kc + (((size_t)blk * MLA_CG + j) * BS + T % BS) * 8),
                                         (__attribute__((address_space(3))) void*)&s.a.t[j][0], 16, 0, 0);
    }
  };
  if ((int)blockIdx.x < nitems) load_tile(mla_item(p, blockIdx.x, NHG));
  if (!wait()) return;
  for (int item = blockIdx.x; item < nitems; item += p.nwg) {
    const MlaItem it = mla_item(p, item, NHG);
    const int b = it.b, c = it.c, pos = it.pos, n = pos + 1;
    const int t0 = c * CHUNK, len = min(CHUNK, n - t0);
    // this launch's positions in the chunk: [nlo, nhi] (decode: pos alone, in the chunk holding it)
    const int nlo = max(first_new(pos), t0), nhi = min(pos, t0 + CHUNK - 1);
    if (item != (int)blockIdx.x) load_tile(it);
    // queries of head hg*GH + wave, in registers: q_c dims lane + 64e (agent-scope loads: written by P1b), and q_pe
    // roped (reference_decode.py:235): lane i < 32 holds dims i (lo) and i + 32 (hi).  The score loop takes each
    // dim's value from its lane with v_readlane: wave-uniform operands with no memory wait in the dependent chain.
    const int j = wave, h = it.hg * GH + j;
    float qv[MLA_KVL / 64], qlo = 0.0f, qhi = 0.0f;
    if (j < GH) {
      const float* qc = qc_of(p, layer, b, h);
#pragma unroll
      for (int e = 0; e < MLA_KVL / 64; ++e) qv[e] = ld_ag(qc + lane + 64 * e);
      if (lane < MLA_R / 2) {
        const float* qp = p.qkv + (size_t)b * p.nqkv + h * MLA_QD + MLA_NOPE;
        const float a0 = ld_ag(qp + 2 * lane), a1 = ld_ag(qp + 2 * lane + 1);
        const float cs = ld_f(p.rope_cos + (size_t)pos * (MLA_R / 2) + lane);
        const float sn = ld_f(p.rope_sin + (size_t)pos * (MLA_R / 2) + lane);
        rope_ds_pair(a0, a1, cs, sn, qlo, qhi);
      }
    }
    // the launch's positions in this chunk: wave NWAVE-1-w builds the latent row of position nlo + w from the QKV
    // output of its row, b - (pos - q) (a launch has at most MAX_B_DS <= NWAVE rows), writes it into the tile slots
    // once the cached rows have landed, and the first head group's item appends the row's own position to the cache
    const int q = nlo + (NWAVE - 1 - wave);
    LatentRow lr;
    if (q <= nhi) lr = latent_row(p, Lw, b - (pos - q), q);
    __builtin_amdgcn_s_waitcnt(0);                        // this wave's tile copies have landed in LDS
    __syncthreads();
    if (q <= nhi) {
      const int tn = q - t0;
      latent_dims(lr, [&](int k, float v) {
        const int jj = k / 8;
        ((uint16_t*)&s.a.t[jj][tn ^ (jj & 15)])[k % 8] = f2bf(v);
      });
      if (q == pos && it.hg == 0) {                       // the cache append (reference_decode.py:236-237)
        const int blk = ld_i(p.btab + (size_t)b * p.nbps + pos / BS), off = pos % BS;
        uint16_t* row = Lw.kc + (size_t)blk * MLA_CG * BS * 8 + off * 8;   // dim k at row + (k / 8) * BS * 8 + k % 8
        latent_dims(lr, [&](int k, float v) { st_u16(row + (size_t)(k / 8) * BS * 8 + k % 8, f2bf(v)); });
      }
    }
    __syncthreads();
    // scores: wave = head, lane = position
    if (j < GH) {
      auto bcast = [](float v, int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l)); };
      float s1 = 0.0f, s2 = 0.0f;
      // tile reads run one block of 4 groups ahead of the fma chain; a group's 8 query values are broadcast first
      constexpr int GB = 4, NB = MLA_CG / GB;
      u32x4 kA[GB], kB[GB];
      auto ld = [&](u32x4(&k)[GB], int blk) {
#pragma unroll
        for (int u = 0; u < GB; ++u) {
          const int g = blk * GB + u;
          k[u] = s.a.t[g][lane ^ (g & 15)];
        }
      };
      auto qdim = [&](int i) -> float {                   // dim i of [q_c; q_pe]
        if (i < MLA_KVL) return bcast(qv[i >> 6], i & 63);
        const int d = i - MLA_KVL;
        return d < MLA_R / 2 ? bcast(qlo, d) : bcast(qhi, d - MLA_R / 2);
      };
      auto acc = [&](const u32x4(&k)[GB], int blk) {
#pragma unroll
        for (int u = 0; u < GB; ++u) {
          const int g = blk * GB + u;
          float q[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) q[e] = qdim(8 * g + e);
          float& sa = g < MLA_KVL / 8 ? s1 : s2;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            sa = __builtin_fmaf(q[2 * e], bf_lo(k[u][e]), sa);
            sa = __builtin_fmaf(q[2 * e + 1], bf_hi(k[u][e]), sa);
          }
        }
      };
      static_assert(NB % 2 == 0 && (MLA_KVL / 8) % GB == 0, "whole blocks, pairs of blocks");
      ld(kA, 0);
#pragma unroll
      for (int blk = 0; blk < NB; blk += 2) {
        ld(kB, blk + 1);
        acc(kA, blk);
        if (blk + 2 < NB) ld(kA, blk + 2);
        acc(kB, blk + 1);
      }
      const bool valid = lane < len;
      const float sc = valid ? (s1 + s2) * p.attn_scale : -__builtin_huge_valf();
      const float m = wave_max(sc);
      s.a.p[j][lane] = valid ? expf_mk(sc - m) : 0.0f;
      if (lane == 0) s.a.m[j] = m;
    }
    __syncthreads();
    // P.V: wave = head, lane = dim group (dims 8 lane .. 8 lane + 7), positions ascending
    if (j < GH) {
      float a[8], l = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = 0.0f;
      const int sw = lane & 15;
      auto step = [&](int t, float pt) {
        const u32x4 cw = s.a.t[lane][t ^ sw];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          a[2 * e] = __builtin_fmaf(pt, bf_lo(cw[e]), a[2 * e]);
          a[2 * e + 1] = __builtin_fmaf(pt, bf_hi(cw[e]), a[2 * e + 1]);
        }
        l = l + pt;
      };
      int t = 0;
      for (; t + 4 <= len; t += 4) {
        const float4 pq = *(const float4*)&s.a.p[j][t];
        step(t, pq.x);
        step(t + 1, pq.y);
        step(t + 2, pq.z);
        step(t + 3, pq.w);
      }
      for (; t < len; ++t) step(t, s.a.p[j][t]);
      float* part = p.apart + (((size_t)b * NH + h) * MAX_CHUNKS + c) * MLA_PART;
#pragma unroll
      for (int e = 0; e < 8; e += 2) st_ag2(part + 8 * lane + e, a[e], a[e + 1]);
      if (lane == 0) st_ag2(part + MLA_KVL, s.a.m[j], l);
    }
    __syncthreads();                                      // the tile and p are free for the next item
  }
}

// P2c: per (sequence b, head h, quarter of its v_head rows): the merge of the chunk partials (M = max m_c,
// w_c = exp(m_c - M), L = sum w_c l_c, A = sum w_c a_c in ascending c, o_c = A / L in fp32), then
// out[b][h*v_head + d] = bfr(W_UV[h][d] . o_c) (reference_decode.py:254-256), the canonical dot of a kv_lora-long
// bf16 row with the fp32 o_c, written as the O projection's lane-permuted bf16 rows.  Thread i merges dim i.
template <int B, class S, class Wait>
__device__ __forceinline__ void phase_wuv_b(const Params& p, int layer, S& s, Wait wait) {
  using WR = Bf16Row<MLA_KVL>;
  constexpr int Q = 4, RQ = MLA_VH / Q, RW = RQ / NWAVE;  // quarters, rows per quarter, rows per wave
  constexpr int CB = 32;                                  // chunks whose partial loads are in flight together
  static_assert(NT == MLA_KVL, "one thread per latent dim");
  const LayerW Lw = layer_w(p, layer);
  const int NH = p.NH, KA = NH * MLA_VH, nitems = p.B * NH * Q;
  const int lane = lane_id(), wave = wave_u(), tid = threadIdx.x;
  float* sw = &s.a.p[0][0];                               // chunk weights w_c
  float* sl = &s.a.p[1][0];                               // chunk sums l_c
  float* xo = s.a.xo;
  typename WR::Regs W[RW];
  auto rows_of = [&](int item, int& b, int& h, int& d0) {
    b = item / (NH * Q);
    const int r = item - b * NH * Q;
    h = r / Q;
    d0 = (r % Q) * RQ + wave * RW;
  };
  auto issue = [&](int item) {
    int b, h, d0;
    rows_of(item, b, h, d0);
#pragma unroll
    for (int k = 0; k < RW; ++k) WR::load(W[k], mrow<WR>(Lw.wuv, (size_t)h * MLA_VH + d0 + k), lane);
  };
  if ((int)blockIdx.x < nitems) issue(blockIdx.x);
  if (!wait()) return;
  for (int item = blockIdx.x; item < nitems; item += p.nwg) {
    int b, h, d0;
    rows_of(item, b, h, d0);
    if (item != (int)blockIdx.x) issue(item);
    const int nch = p.posb[b] / CHUNK + 1;
    const float* part = p.apart + ((size_t)b * NH + h) * MAX_CHUNKS * MLA_PART;
    float av[CB];
    auto load_a = [&](int c0) {
#pragma unroll
      for (int u = 0; u < CB; ++u) av[u] = ld_ag(part + (size_t)min(c0 + u, nch - 1) * MLA_PART + tid);
    };
    load_a(0);
    if (wave == 0) {                                      // chunk weights and sums (lane c holds chunks c, c + 64)
      float m0 = -__builtin_huge_valf(), l0 = 0.0f, m1 = -__builtin_huge_valf(), l1 = 0.0f;
      if (lane < nch) ld_ag2(part + (size_t)lane * MLA_PART + MLA_KVL, m0, l0);
      if (lane + 64 < nch) ld_ag2(part + (size_t)(lane + 64) * MLA_PART + MLA_KVL, m1, l1);
      const float M = wave_max(fmaxf(m0, m1));
      sw[lane] = lane < nch ? expf_mk(m0 - M) : 0.0f;
      sw[64 + lane] = lane + 64 < nch ? expf_mk(m1 - M) : 0.0f;
      sl[lane] = l0;
      sl[64 + lane] = l1;
    }
    __syncthreads();
    float A = 0.0f, L = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += CB) {
      if (c0 > 0) load_a(c0);
#pragma unroll
      for (int u = 0; u < CB; ++u)
        if (c0 + u < nch) {
          const float wc = sw[c0 + u];
          L = __builtin_fmaf(wc, sl[c0 + u], L);
          A = __builtin_fmaf(wc, av[u], A);
        }
    }
    xo[perm_stored(tid, MLA_KVL)] = A / L;
    __syncthreads();
    const float4 x0 = *(const float4*)&xo[8 * lane], x1 = *(const float4*)&xo[8 * lane + 4];
#pragma unroll
    for (int k = 0; k < RW; ++k) {
      const u32x4 w = W[k].w[0];
      float acc = 0.0f;
      acc = __builtin_fmaf(bf_lo(w[0]), x0.x, acc);
      acc = __builtin_fmaf(bf_hi(w[0]), x0.y, acc);
      acc = __builtin_fmaf(bf_lo(w[1]), x0.z, acc);
      acc = __builtin_fmaf(bf_hi(w[1]), x0.w, acc);
      acc = __builtin_fmaf(bf_lo(w[2]), x1.x, acc);
      acc = __builtin_fmaf(bf_hi(w[2]), x1.y, acc);
      acc = __builtin_fmaf(bf_lo(w[3]), x1.z, acc);
      acc = __builtin_fmaf(bf_hi(w[3]), x1.w, acc);
      acc = wave_sum(acc);
      if (lane == 0) st_ag_u16(p.o16 + (size_t)b * KA + perm_stored(h * MLA_VH + d0 + k, KA), f2bf(acc));
    }
    __syncthreads();                                      // xo, sw, sl are free for the next item
  }
}

// P4: post-attention RMSNorm, then one GEMV over the router rows (fp32 logits, not rounded: reference_decode.py:271)
// and the shared experts' interleaved gate/up rows (SiLU(g) * u into h16s, :286 with mlp_unit :259-265)
template <int KK, int B, class S, class Wait>
__device__ __forceinline__ void phase_router_shared_b(const Params& p, int layer, S& s, Wait wait) {
  using WR = Bf16Row<KK>;
  const LayerW Lw = layer_w(p, layer);
  const int E = p.E, E2 = E / 2, SI = p.SI, nb = p.B;
  gemv_run_b<WR, 2, B>(
      E2 + SI,
      [&](int g, int i) -> const uint8_t* {
        return g < E2 ? mrow<WR>(Lw.wr, (size_t)2 * g + i) : mrow<WR>(Lw.wsgu, (size_t)2 * (g - E2) + i);
      },
      [&](int) { return nb; }, [&](int, int b) { return (const uint16_t*)(s.n.xs + b * KK); },
      [&](int g, int nv, const float(&v)[2][B]) {
        if (g < E2) {
          lane_store_b<2, B>(v, nv, [&](int i, int b, float val, bool ok) {
            st_ag(ok ? p.logits + (size_t)b * E + 2 * g + i : sink_of(p), val);
          });
        } else {
          const int j = g - E2, lane = lane_id();
          const float gv = lane_pick<1, B>((const float(&)[1][B])v[0]), uv = lane_pick<1, B>((const float(&)[1][B])v[1]);
          st_ag_u16(lane < nv ? p.h16s + (size_t)lane * SI + perm_stored(j, SI) : (uint16_t*)sink_of(p),
                    f2bf(bfr(bfr(silu(bfr(gv))) * bfr(uv))));
        }
      },
      [&]() {
        if (!wait()) return false;
        build_norm_xb<KK, B>(p, false, Lw.ln2, s);
        return true;
      },
      p.nwg, p.trace, s.phase);
}

// P6: routed experts' down rows, y = bfr(w * bfr(W2[e] . h)) per routed pair, summed in fp32 in ascending expert id
// per sequence (reference_decode.py:280-284), plus the shared experts' down row sh = bfr(W_sd . h_s) (:286):
// x = bfr(x + bfr(bfr(y) + sh)) (:287, :302).  The routing (and its pair lists) is P5's, kept in LDS; all pairs'
// and the shared h rows fit LDS at once.
template <int KM, int KSH, int B, class S, class Wait>
__device__ __forceinline__ void phase_ds_down_b(const Params& p, int layer, S& s, Wait wait) {
  using WR = Bf16Row<KM>;
  using WS = Bf16Row<KSH>;
  constexpr int DE = WR::REGS <= 7 ? 8 : WR::REGS <= 13 ? 4 : 2;
  static_assert(B * MAX_TOPK * KM + B * KSH <= S::XCAP, "expert rows exceed the LDS budget");
  using Regs = typename WR::Regs;
  const LayerW Lw = layer_w(p, layer);
  const int H = p.H, nb = p.B, nw = p.nwg * NWAVE, lane = lane_id();
  const int gw = blockIdx.x * NWAVE + wave_u();
  const int U = s.nexp, np = s.ustart[U];
  const int nrw = gw < H ? (H - 1 - gw) / nw + 1 : 0;    // output rows of this wave
  const int nbt = (U + DE - 1) / DE, T = nrw * nbt;
  typename WS::Regs RS[1];
  Regs R[2][DE];
  auto issue = [&](Regs(&Rb)[DE], int t) {
    const int g = gw + (t / nbt) * nw, ub = (t % nbt) * DE;
#pragma unroll
    for (int d = 0; d < DE; ++d)
      if (ub + d < U) WR::load(Rb[d], mrow<WR>(Lw.w2, (size_t)s.uexp[ub + d] * H + g), lane);
  };
  if (nrw > 0) WS::load(RS[0], mrow<WS>(Lw.wsd, gw), lane);
  if (T > 0) issue(R[0], 0);
  if (p.trace && threadIdx.x == 0)
    *(MK_G uint64_t*)(p.trace + ((size_t)s.phase * p.nwg + blockIdx.x) * 3 + 2) = __builtin_amdgcn_s_memrealtime();
  load_res_rows<B>(p, H, false, s);
  if (!wait()) return;
  uint16_t* hs = s.v.xs + (size_t)np * KM;                // shared rows after the pairs' rows
  copy_rows_lds(p.h16, np * KM, s.v.xs);
  copy_rows_lds(p.h16s, nb * KSH, hs);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int k = 0; k < nrw; ++k) {                         // shared down of every output row of this wave
    const int g = gw + k * nw;
    if (k > 0) WS::load(RS[0], mrow<WS>(Lw.wsd, g), lane);
    float v[1][B];
    dot_rows_b<KSH, 1, B>(RS, [&](int b) { return (const uint16_t*)(hs + b * KSH); }, nb, lane, v);
    float mine = 0.0f;
#pragma unroll
    for (int b = 0; b < B; ++b)
      if (lane == b) mine = v[0][b];
    if (lane < nb) s.v.sh[lane][res_slot(g, nw)] = bfr(mine);
  }
  float acc = 0.0f;
  auto compute = [&](Regs(&Rb)[DE], int t) {
    const int g = gw + (t / nbt) * nw, ub = (t % nbt) * DE, r = res_slot(g, nw);
    if (t % nbt == 0) acc = 0.0f;
#pragma unroll
    for (int d = 0; d < DE; ++d)
      if (ub + d < U)
        for (int pp = s.ustart[ub + d]; pp < s.ustart[ub + d + 1]; ++pp) {
          const float y = bfr(s.pw[pp] * bfr(WR::dot(Rb[d], s.v.xs + (size_t)pp * KM, lane)));
          if (lane == s.pseq[pp]) acc = acc + y;
        }
    if (t % nbt == nbt - 1 && lane < nb)
      st_ag_u16(p.x16 + (size_t)lane * H + g, f2bf(s.v.xres[lane][r] + bfr(bfr(acc) + s.v.sh[lane][r])));
  };
  for (int t = 0; t < T; t += 2) {
    if (t + 1 < T) issue(R[1], t + 1);
    compute(R[0], t);
    if (t + 2 < T) issue(R[0], t + 2);
    if (t + 1 < T) compute(R[1], t + 1);
  }
}

// ---------------------------------------------------------------- DeepSeek-V2 persistent kernel
// H hidden, KA = NH * v_head, KM routed expert width, KSH shared width (n_shared * KM), EC experts, IP dense width
// rounded up to the row format, B batch capacity
template <int H, int KA, int KM, int KSH, int EC, int IP>
struct DsCap {
  static constexpr int a = MAX_B_DS * (MAX_TOPK * KM + KSH), b = MAX_B_DS * IP, c = MAX_B_DS * KA;
  static constexpr int d = MAX_B_DS * MLA_MAX_NH * MLA_NOPE, e = MAX_B_DS * 2 * MLA_KVL * 2;
  static constexpr int m1 = a > b ? a : b, m2 = c > d ? c : d, m3 = m1 > m2 ? m1 : m2;
  static constexpr int value = m3 > e ? m3 : e;
};

template <int H, int KA, int KM, int KSH, int EC, int IP, int B>
__device__ __forceinline__ void fused_body_ds(const Params& p) {
  __shared__ SmemD<B, DsCap<H, KA, KM, KSH, EC, IP>::value> s;
  if (threadIdx.x == 0) s.abort = 0;
  __syncthreads();
  int k = 0;
  auto wait = [&]() { return grid_wait(p, k, s); };
  if (p.trace && threadIdx.x == 0) *(MK_G uint64_t*)(p.trace + (size_t)blockIdx.x * 3) = __builtin_amdgcn_s_memrealtime();
  s.phase = 0;
  for (int layer = p.l0; layer < p.l1; ++layer) {
    phase_qkv_b<Bf16Row<H>, B>(p, layer, s, wait);
    if (s.abort) return;
    grid_arrive(p, k, s);
    phase_absorb_b<B>(p, layer, s, wait);
    if (s.abort) return;
    grid_arrive(p, k, s);
    phase_mla_attn<B>(p, layer, s, wait);
    if (s.abort) return;
    grid_arrive(p, k, s);
    phase_wuv_b<B>(p, layer, s, wait);
    if (s.abort) return;
    grid_arrive(p, k, s);
    phase_oproj_b<Bf16Row<KA>, B>(p, layer, s, wait);
    if (s.abort) return;
    grid_arrive(p, k, s);
    if (layer < p.first_dense) {
      phase_gateup_b<Bf16Row<H>, B>(p, layer, s, wait);
      if (s.abort) return;
      grid_arrive(p, k, s);
      phase_down_b<Bf16Row<IP>, B>(p, layer, s, wait);
      if (s.abort) return;
      grid_arrive(p, k, s);
    } else {
      phase_router_shared_b<H, B>(p, layer, s, wait);
      if (s.abort) return;
      grid_arrive(p, k, s);
      phase_expert_up_b<Bf16Row<H>, B, EC>(p, layer, s, wait);
      if (s.abort) return;
      grid_arrive(p, k, s);
      phase_ds_down_b<KM, KSH, B>(p, layer, s, wait);
      if (s.abort) return;
      grid_arrive(p, k, s);
    }
  }
  if (p.do_head) {
    phase_head_b<H, B>(p, s, wait);
    if (s.abort) return;
    grid_arrive(p, k, s);
    phase_token_b(p, wait);
  }
}

// DeepSeek-V2 shapes: name, H, NH*v_head, MI, n_shared*MI, E, dense I rounded up to 512, batch capacity
#define MK_DS_SHAPES(X)                                                                        \
  X(etxmk_ds_b4_h2048_a2048_moe1408_s2816_e64_d11264, 2048, 2048, 1408, 2816, 64, 11264, 4) \
  X(etxmk_ds_b4_h512_a512_moe256_s512_e16_d1024, 512, 512, 256, 512, 16, 1024, 4)
#define MK_DS_KERNEL(name, H, KA, KM, KSH, EC, IP, B) \
  extern "C" __global__ void __launch_bounds__(NT, 1) name(Params p) { fused_body_ds<H, KA, KM, KSH, EC, IP, B>(p); }
#define MK_DS_DECL(name, H, KA, KM, KSH, EC, IP, B) extern "C" __global__ void __launch_bounds__(NT, 1) name(Params p);

}  // namespace mk
