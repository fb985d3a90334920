#pragma once
// Batched decode step: B sequences (at most MAX_B) per persistent launch, each at its own position with its own
// paged-KV block table and token row.  The phases are those of the single-sequence kernel (mk_device.h); every
// weight row streams from HBM once per step and is dotted with the input vectors of every sequence that needs it.
// Per (row, sequence) the arithmetic is the single-sequence dot in the same order, so a batched step equals B
// single-sequence steps bit for bit.  Handles of batch capacity >= 8 whose shapes take whole tiles (Params.mfma, the
// host's matrix-core rule) run the dense projections, the router, the experts and the lm_head instead as tiles of 16
// weight rows against up to 16 sequence columns on v_mfma_f32_16x16x32_bf16: each (row, sequence) value is then the
// matrix-core chain in a fixed order (per form below), the same for every column, so a batched step still equals B
// single steps of the CPU oracle stated with the same rule.
//
// Reference path: examples/vllm_llm/host.hip:126-1159 and examples/vllm_llm/vl_tiles.hip:1-95 (per-request
// parameters, block tables, slot mapping, greedy argmax), with examples/llm/ref_numpy.py:105-158 per sequence.
//
// Activations between phases (global memory, one row per sequence):
//   x16     [B][H] bf16       residual (its values are bf16 in every case, so storing them as bf16 rounds nothing)
//   qkv     [B][NQKV] fp32    as in the single-sequence kernel
//   o16     [B][NH*HD] bf16   attention output, lane-permuted: the O projection copies rows straight into LDS
//   logits  [B][E] fp32       router logits
//   h16     MoE [pairs][MI] / dense [B][I] bf16, lane-permuted; MoE rows are the routed (sequence, slot) pairs in
//           pair order (ascending expert, then sequence); with the matrix cores and fp8 weights, in the fp8 rows'
//           stored order (blocks of 1024) that the down tiles chain over
//   ys      [pairs][H] bf16   matrix-core expert down: each pair's weighted outputs, added per sequence by the
//           combine phase
// Cross-workgroup values are written with agent-scope stores and read with agent-scope loads (sc1), as in the
// single-sequence kernel.
#include "mk_device.h"

namespace mk {

constexpr int RES_ROWS = 64;            // residual rows per workgroup and sequence held for the epilogues
constexpr int MAX_PAIRS = MAX_B * MAX_TOPK;
constexpr int KEY_WORDS = MAX_E * MAX_B / 32;  // routed-pair keys expert * MAX_B + sequence, one bit each
constexpr int ATTN_CPI_B = 2;           // chunks per attention item in batched kernels

typedef __bf16 mk_bf16x8 __attribute__((ext_vector_type(8)));   // MFMA operands, accumulators
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float mk_f32x4 __attribute__((ext_vector_type(4)));

// LDS of the batched attention phase: two buffers of ATTN_CPI_B chunk tile pairs (the next item's K and V stream in
// while this item computes); the merge phase's per-wave chunk weights and sums
struct AttnTilesB {
  u32x4 kt[2][ATTN_CPI_B][HDIM / 8][CHUNK];         // [buffer][chunk][8-dim group][position]
  u32x4 vt[2][ATTN_CPI_B][CHUNK / 8][2][CHUNK];     // [buffer][chunk][8-position group][dim half][dim in half]
  // wave j's roped q (dims in order) and its chunks' probabilities (positions in order), read back by the whole wave
  // at one address (an LDS broadcast) as the wave-uniform operands of the score and P.V chains
  alignas(16) float qb[NWAVE][HDIM];
  alignas(16) float pb[NWAVE][ATTN_CPI_B][CHUNK];
};
struct AttnMergeB {
  float p[NWAVE][2 * MAX_CHUNKS];
};

template <int B>
struct SmemB {
  static constexpr int NCAP = B * MAX_H > 32768 ? 32768 : B * MAX_H;    // B * H of the norm phases
  static constexpr bool NORM_HOIST = true;              // build_norm_xb loads a thread's weights once
  static constexpr int XCAP = B * MAX_K > 65536 ? 65536 : B * MAX_K;    // input rows of the other GEMVs
  union {
    struct {
      alignas(16) uint16_t xr[NCAP];    // residual rows, natural order
      alignas(16) uint16_t xs[NCAP];    // normed rows, lane-permuted
    } n;
    struct {
      alignas(16) uint16_t xs[XCAP];    // input rows (o, h), lane-permuted
      float xres[B][RES_ROWS];          // residual of this workgroup's output rows
      float acc[B][RES_ROWS];           // expert combine carried from one pass over the pairs to the next
    } v;
    AttnTilesB a;
    AttnMergeB m;
  };
  float rs[B];                          // 1/rms per sequence
  int32_t rids[B][MAX_TOPK];            // routing per sequence, slot order
  float rwts[B][MAX_TOPK];
  int32_t pexp[MAX_PAIRS];              // routed pairs sorted by (expert, sequence): expert, sequence, weight
  int32_t pseq[MAX_PAIRS];
  float pw[MAX_PAIRS];
  int32_t uexp[MAX_PAIRS];              // distinct experts ascending; expert u owns pairs [ustart[u], ustart[u + 1])
  int32_t ustart[MAX_PAIRS + 1];
  int32_t nexp;
  int32_t bpair[B][MAX_TOPK];           // sequence b's pairs (indices into pexp..) in ascending expert order
  uint32_t kbits[KEY_WORDS];            // routing: bitmap of the pairs' keys, then their prefix popcounts
  uint32_t kpre[KEY_WORDS];
  int32_t abort, last, phase;
};

__device__ __forceinline__ int token_of_b(const Params& p, int b) {
  const int t = ld_ag_i(p.tokens + (size_t)b * p.tok_stride + p.posb[b]);
  return (t >= 0 && t < p.V) ? t : 0;
}

// nelem bf16 (global, contiguous, a multiple of 8) -> dst (LDS), 16 bytes per lane, agent-coherent.  Lane l of a
// wave writes the 16 bytes after its wave's base, so each wave copies 64 consecutive chunks per round.
__device__ __forceinline__ void copy_rows_lds(const uint16_t* src, int nelem, uint16_t* dst) {
  const int lane = lane_id(), nch = nelem / 8;
  for (int c0 = wave_u() * 64; c0 < nch; c0 += NT)
    if (c0 + lane < nch)
      __builtin_amdgcn_global_load_lds((const MK_G void*)(src + 8 * (c0 + lane)),
                                       (__attribute__((address_space(3))) void*)(dst + 8 * c0), 16, 0, LDS_SC1);
}

// The residual rows -> s.n.xr (bf16, natural order): the embedding rows of the sequences' tokens for the first
// layer, else x16.  Then per sequence r = 1/sqrt(mean(x^2) + eps) with the sum of squares in dot order, and the
// normed lane-permuted rows bfr(w * bfr(x * r)) -> s.n.xs (ref_numpy.py:71-73, as build_norm_x).  Thread t normalises
// the 8 consecutive elements of chunk t % (H/8) in rows t / (H/8), t / (H/8) + 512 / (H/8), ...: one 16-byte read of
// x and of w, eight 2-byte writes to their permuted positions.
template <int H, int B, class S>
__device__ __forceinline__ void build_norm_xb(const Params& p, bool first, const uint16_t* w, S& s) {
  static_assert(B * H <= S::NCAP, "residual rows exceed the LDS budget");
  constexpr int C8 = H / 8, RSTEP = NT / C8;
  static_assert(NT % C8 == 0, "a workgroup covers whole rows of chunks");
  const int nb = p.B, lane = lane_id(), wave = wave_u();
  const int c = (int)threadIdx.x % C8, b0 = (int)threadIdx.x / C8;
  const u32x4 wv = ld16(w + 8 * c);
  constexpr int NS = H / 8;
  // slot form (H a multiple of 512) with whole rows of slots per workgroup: thread t writes slot t % NS of every
  // row, so its 8 weights are loaded once, with the row copy, instead of once per row after it (8 more live VGPRs
  // across the copy: layouts whose kernels are short of registers set NORM_HOIST false and keep the per-row loads)
  constexpr bool FIXED = S::NORM_HOIST && H % 512 == 0 && NT % NS == 0;
  uint16_t wk[8];
  if constexpr (FIXED) {
    const int sl = (int)threadIdx.x % NS, base = 512 * (sl >> 6), l = sl & 63;
#pragma unroll
    for (int j = 0; j < 8; ++j) wk[j] = ld_u16(w + base + l + 64 * j);
  }
  if (first) {
    for (int q = threadIdx.x; q < nb * C8; q += NT) {
      const int b = q / C8, qq = q - b * C8;
      *(u32x4*)(s.n.xr + 8 * q) = ld16(p.embed + (size_t)token_of_b(p, b) * H + 8 * qq);
    }
  } else {
    copy_rows_lds(p.x16, nb * H, s.n.xr);
    __builtin_amdgcn_s_waitcnt(0);
  }
  __syncthreads();
  for (int b = wave; b < nb; b += NWAVE) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < H / 64; ++i) {
      const float v = bf2f(s.n.xr[b * H + lane + 64 * i]);
      acc = __builtin_fmaf(v, v, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) s.rs[b] = 1.0f / __builtin_sqrtf(acc / (float)H + p.eps);
  }
  __syncthreads();
  if constexpr (H % 512 == 0) {
    // thread t writes whole 16-byte slots of the lane-permuted rows: slot (b, block, lane l) holds the logical
    // elements 512 block + l + 64 j, j < 8, read from the natural rows (consecutive lanes read consecutive elements,
    // write consecutive slots: no LDS bank conflicts; scattered 2-byte writes put 16 lanes on each bank)
    for (int t = threadIdx.x; t < nb * NS; t += NT) {    // NS slots per row
      const int b = t / NS, sl = t - b * NS, base = 512 * (sl >> 6), l = sl & 63;
      const float r = s.rs[b];
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int k0 = base + l + 64 * (2 * e), k1 = k0 + 64;
        const float w0 = bf2f(FIXED ? wk[2 * e] : ld_u16(w + k0)), w1 = bf2f(FIXED ? wk[2 * e + 1] : ld_u16(w + k1));
        const float y0 = bfr(w0 * bfr(bf2f(s.n.xr[b * H + k0]) * r));
        const float y1 = bfr(w1 * bfr(bf2f(s.n.xr[b * H + k1]) * r));
        o[e] = (uint32_t)f2bf(y0) | ((uint32_t)f2bf(y1) << 16);
      }
      *(u32x4*)(s.n.xs + b * H + 8 * sl) = u32x4{o[0], o[1], o[2], o[3]};
    }
  } else {
    for (int b = b0; b < nb; b += RSTEP) {
      const float r = s.rs[b];
      const u32x4 xv = *(const u32x4*)(s.n.xr + b * H + 8 * c);
      uint16_t* dst = s.n.xs + b * H;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int k = 8 * c + 2 * e;
        dst[perm_stored(k, H)] = f2bf(bfr(bf_lo(wv[e]) * bfr(bf_lo(xv[e]) * r)));
        dst[perm_stored(k + 1, H)] = f2bf(bfr(bf_hi(wv[e]) * bfr(bf_hi(xv[e]) * r)));
      }
    }
  }
  __syncthreads();
}

// Residual entries of this workgroup's output rows for the NR = 1 phases (O projection, down projections): row
// g = d*nw + 8*blockIdx.x + i is wave i's row of round d and lands in xres[b][8*d + i].  Read before the phase's
// wait: the residual was last written at least two barriers earlier.
template <int B, class S>
__device__ __forceinline__ void load_res_rows(const Params& p, int nrows, bool first, S& s) {
  const int nw = p.nwg * NWAVE, per = ((nrows + nw - 1) / nw) * NWAVE;
  for (int t = threadIdx.x; t < p.B * per; t += NT) {
    const int b = t / per, r = t - b * per;
    const int g = (r / NWAVE) * nw + (int)blockIdx.x * NWAVE + r % NWAVE;
    if (g < nrows)
      s.v.xres[b][r] = first ? bf2f(ld_u16(p.embed + (size_t)token_of_b(p, b) * p.H + g))
                             : bf2f(ld_ag_u16(p.x16 + (size_t)b * p.H + g));
  }
}
// the xres slot of row g for the calling wave
__device__ __forceinline__ int res_slot(int g, int nw) { return (g / nw) * NWAVE + wave_u(); }

// NR rows (in registers) dotted with up to B input rows in LDS (xp(b), b < nv; nv is wave-uniform).  For each
// (row, input) the lane accumulates its elements in ascending order exactly as dot_row does, then wave_sum.
template <int K, int NR, int B, class XP>
__device__ __forceinline__ void dot_rows_b(const RowRegs<K> (&r)[NR], XP xp, int nv, int lane, float (&v)[NR][B]) {
  float acc[NR][B];
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int b = 0; b < B; ++b) acc[i][b] = 0.0f;
#pragma unroll
  for (int blk = 0; blk < KS<K>::KB; ++blk) {
#pragma unroll
    for (int b = 0; b < B; ++b)
      if (b < nv) {
        const u32x4 xv = *(const u32x4*)(xp(b) + 512 * blk + lane * 8);
#pragma unroll
        for (int i = 0; i < NR; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[i][b] = __builtin_fmaf(bf_lo(r[i].w[blk][j]), bf_lo(xv[j]), acc[i][b]);
            acc[i][b] = __builtin_fmaf(bf_hi(r[i].w[blk][j]), bf_hi(xv[j]), acc[i][b]);
          }
      }
  }
#pragma unroll
  for (int t = 0; t < KS<K>::TW; ++t) {
#pragma unroll
    for (int b = 0; b < B; ++b)
      if (b < nv) {
        const uint32_t xv = *(const uint32_t*)(xp(b) + 512 * KS<K>::KB + lane * KS<K>::TM + 2 * t);
#pragma unroll
        for (int i = 0; i < NR; ++i) {
          acc[i][b] = __builtin_fmaf(bf_lo(r[i].t[t]), bf_lo(xv), acc[i][b]);
          acc[i][b] = __builtin_fmaf(bf_hi(r[i].t[t]), bf_hi(xv), acc[i][b]);
        }
      }
  }
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int b = 0; b < B; ++b) v[i][b] = b < nv ? wave_sum(acc[i][b]) : 0.0f;
}

// a long row (Bf16Row LONG) dotted with up to B input rows: dot_row_long's segments, each block's weights used for
// every input, per (row, input) the order of dot_row
template <int K, int B, class XP>
__device__ __forceinline__ void dot_row_long_b(const uint16_t* row, XP xp, int nv, int lane, float (&v)[B]) {
  constexpr int SEG = seg_of(KS<K>::KB), NS = SEG ? KS<K>::KB / SEG : 0;
  static_assert(SEG > 0 && KS<K>::TW == 0, "long rows are whole segments of 4 to 12 blocks");
  u32x4 RA[SEG], RB[SEG];
  float acc[B];
#pragma unroll
  for (int b = 0; b < B; ++b) acc[b] = 0.0f;
  auto ld = [&](u32x4(&R)[SEG], int sg) {
#pragma unroll
    for (int k = 0; k < SEG; ++k) R[k] = ld_nt16(row + 512 * (sg * SEG + k) + lane * 8);
  };
  auto acc_seg = [&](const u32x4(&R)[SEG], int sg) {
#pragma unroll
    for (int k = 0; k < SEG; ++k)
#pragma unroll
      for (int b = 0; b < B; ++b)
        if (b < nv) {
          const u32x4 xv = *(const u32x4*)(xp(b) + 512 * (sg * SEG + k) + lane * 8);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[b] = __builtin_fmaf(bf_lo(R[k][j]), bf_lo(xv[j]), acc[b]);
            acc[b] = __builtin_fmaf(bf_hi(R[k][j]), bf_hi(xv[j]), acc[b]);
          }
        }
  };
  ld(RA, 0);
#pragma unroll 1
  for (int sg = 0; sg < NS; sg += 2) {
    if (sg + 1 < NS) ld(RB, sg + 1);
    acc_seg(RA, sg);
    if (sg + 2 < NS) ld(RA, sg + 2);
    if (sg + 1 < NS) acc_seg(RB, sg + 1);
  }
#pragma unroll
  for (int b = 0; b < B; ++b) v[b] = b < nv ? wave_sum(acc[b]) : 0.0f;
}

// the wave's store sink: the target of epilogue lanes that have no value to store.  All of them write the same
// word (one of the values lands; the line written is one per store, not four); waves are 256 bytes apart.
__device__ __forceinline__ float* sink_of(const Params& p) {
  return p.sink + (size_t)((blockIdx.x * NWAVE + wave_u()) & (SINK_WAVES - 1)) * 64;
}

// gemv_run with B input rows per group: groups of NR rows dealt round-robin to the grid's waves.  D register buffers
// form a ring: the next D - 1 groups' weights stream while one group is reduced, the first D - 1 issued before
// `prologue` (which waits for the inputs).  Every issue is the same run of loads: a missing row (nullptr) reloads
// the group's first row, and past the wave's last group the issues reload that group (non-temporal loads, so these
// are fetched from HBM again, not served from the cache: the price of an exact wait count); with epilogues of
// one store per lane (the sink for lanes with nothing to store) the compiler's wait before a buffer's dots counts
// exactly the loads and stores issued after it, so it never waits for groups still streaming.  nvec(g) is the number
// of input rows of group g, xvec(g, b) the LDS address of its b-th; epi(g, nv, v) consumes v[NR][B].
template <class WR, int NR, int B, int D = 2, class RowF, class NVF, class XF, class EpiF, class Pro>
__device__ __forceinline__ bool gemv_run_b(int ngroups, RowF rowf, NVF nvec, XF xvec, EpiF epi, Pro prologue, int nwg,
                                           uint64_t* trace, int s_phase) {
  using Regs = typename WR::Regs;
  static_assert(D >= 2, "a ring of at least two buffers");
  const int lane = lane_id();
  const int gw = blockIdx.x * NWAVE + wave_u(), nw = nwg * NWAVE;
  if constexpr (WR::LONG) {                               // rows streamed in segments (dot_row_long_b)
    if (!prologue()) return false;
    for (int g = gw; g < ngroups; g += nw) {
      const int nv = nvec(g);
      float v[NR][B];
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        const uint8_t* rp = rowf(g, i);
        if (rp) dot_row_long_b<WR::K, B>((const uint16_t*)rp, [&](int b) { return xvec(g, b); }, nv, lane, v[i]);
        else
#pragma unroll
          for (int b = 0; b < B; ++b) v[i][b] = 0.0f;
      }
      epi(g, nv, v);
    }
    return true;
  } else {
    Regs R[D][NR];
    const bool any = gw < ngroups;
    const int last = any ? gw + (ngroups - 1 - gw) / nw * nw : 0;
    auto issue = [&](Regs(&Rb)[NR], int g) {             // the lane per issue and per compute, held by neither
      const int gc = g <= last ? g : last, lane = lane_id();
      const uint8_t* r0 = rowf(gc, 0);
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        const uint8_t* rp = i == 0 ? r0 : rowf(gc, i);
        WR::load(Rb[i], rp ? rp : r0, lane);
      }
    };
    auto compute = [&](const Regs(&Rb)[NR], int g) {
      const int nv = nvec(g), lane = lane_id();
      float v[NR][B];
      dot_rows_any<WR, NR, B>(Rb, [&](int b) { return xvec(g, b); }, nv, lane, v);
      epi(g, nv, v);
    };
    auto stamp = [&]() {
      if (trace && threadIdx.x == 0)
        *(MK_G uint64_t*)(trace + ((size_t)s_phase * nwg + blockIdx.x) * 3 + 2) = __builtin_amdgcn_s_memrealtime();
    };
    const int n = any ? (last - gw) / nw + 1 : 0;        // this wave's groups
    if (n == 1 || n == 2) {                               // one or two groups: no ring, no reloads
      issue(R[0], gw);
      stamp();
      if (!prologue()) return false;
      if (n == 2) issue(R[1], gw + nw);
      compute(R[0], gw);
      if (n == 2) compute(R[1], gw + nw);
      return true;
    }
    if (any)
#pragma unroll
      for (int j = 0; j + 1 < D; ++j) issue(R[j], gw + j * nw);
    stamp();
    if (!prologue()) return false;
    if (!any) return true;
    issue(R[D - 1], gw + (D - 1) * nw);                   // the last slot after the wait: more loads in flight
    int g = gw;                                           // during the grid barrier slow the barrier down
    for (;;) {                                            // a buffer is refilled right after its dots: the issue's
#pragma unroll                                            // address temporaries alias no load still in flight
      for (int j = 0; j < D; ++j) {
        compute(R[j], g);
        if (g >= last) goto done;
        issue(R[j], g + D * nw);
        g += nw;
      }
    }
  done:
    return true;
  }
}

// fp8 rows (Fp8Row) dotted with up to B input rows: each block's codes are decoded once and used for every input;
// per (row, input) the order is dot_row8's, then wave_sum and the row's scale
template <int K, int NR, int B, class XP>
__device__ __forceinline__ void dot_rows_b8(const RowRegs8<K> (&r)[NR], XP xp, int nv, int lane, float (&v)[NR][B]) {
  constexpr int NB = KS8<K>::KB + (KS8<K>::T > 0 ? 1 : 0);
  float acc[NR][B];
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int b = 0; b < B; ++b) acc[i][b] = 0.0f;
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int n = j < KS8<K>::KB ? 16 : KS8<K>::TM;
    float wv[NR][16];
#pragma unroll
    for (int i = 0; i < NR; ++i) w_of_fp8_block<K>(r[i], j, wv[i]);
#pragma unroll
    for (int b = 0; b < B; ++b)
      if (b < nv) {
        float xv[16];
        x_of_fp8_block<K>(xp(b), j, lane, xv);
#pragma unroll
        for (int i = 0; i < NR; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (e < n) acc[i][b] = __builtin_fmaf(wv[i][e], xv[e], acc[i][b]);
      }
  }
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int b = 0; b < B; ++b) v[i][b] = b < nv ? wave_sum(acc[i][b]) * r[i].sc : 0.0f;
}

template <class WR, int NR, int B, class XP>
__device__ __forceinline__ void dot_rows_any(const typename WR::Regs (&r)[NR], XP xp, int nv, int lane, float (&v)[NR][B]) {
  if constexpr (WR::FP8) dot_rows_b8<WR::K, NR, B>(r, xp, nv, lane, v);
  else dot_rows_b<WR::K, NR, B>(r, xp, nv, lane, v);
}

// value (i, b) of v[NR][B] (wave-uniform) selected into lane i*B + b; other lanes get 0
template <int NR, int B>
__device__ __forceinline__ float lane_pick(const float (&v)[NR][B]) {
  const int lane = lane_id();
  float r = 0.0f;
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int b = 0; b < B; ++b)
      if (i * B + b < 64) r = lane == i * B + b ? v[i][b] : r;
  return r;
}
// store NR x B values: lane i*B + b holds (i, b), valid for i < NR and b < nv; f(i, b, val, ok) makes one store
// from every lane, to the sink where !ok
template <int NR, int B, class F>
__device__ __forceinline__ void lane_store_b(const float (&v)[NR][B], int nv, F f) {
  static_assert(NR * B <= 64, "one lane per value");
  const int lane = lane_id(), i = lane / B, b = lane - i * B;
  const float val = lane_pick<NR, B>(v);
  f(i < NR ? i : 0, b, val, i < NR && b < nv);
}

// ---------------------------------------------------------------- phases (batched)
// P1: input RMSNorm + QKV GEMV per sequence (ref_numpy.py:111-115)
template <class WR, int B, class S, class Wait>
__device__ __forceinline__ void phase_qkv_b(const Params& p, int layer, S& s, Wait wait) {
  constexpr int KK = WR::K;
  const LayerW Lw = layer_w(p, layer);
  const bool first = layer == p.l0 && p.do_embed;
  const int rows = p.nqkv, nb = p.B;
  const uint8_t* W = Lw.wqkv;
  gemv_run_b<WR, 2, B>(
      (rows + 1) / 2,
      [&](int g, int i) -> const uint8_t* { const int r = 2 * g + i; return r < rows ? mrow<WR>(W, r) : nullptr; },
      [&](int) { return nb; }, [&](int, int b) { return (const uint16_t*)(s.n.xs + b * KK); },
      [&](int g, int nv, const float(&v)[2][B]) {
        lane_store_b<2, B>(v, nv, [&](int i, int b, float val, bool ok) {
          const int r = 2 * g + i;
          st_ag(ok && r < rows ? p.qkv + (size_t)b * rows + r : sink_of(p), bfr(val));
        });
      },
      [&]() {
        if (!wait()) return false;
        build_norm_xb<KK, B>(p, first, Lw.ln1, s);
        if (blockIdx.x == 0) {
          if (p.dump_x && layer > p.l0)
            for (int i = threadIdx.x; i < nb * KK; i += NT)
              st_f(p.dump_x + (size_t)(layer - 1) * nb * KK + i, bf2f(s.n.xr[i]));
          if (layer == p.l0 && p.do_head && (int)threadIdx.x < nb)
            __hip_atomic_store(p.amax + 32 * threadIdx.x, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return true;
      },
      p.nwg, p.trace, s.phase);
}

// P2 (batched): chunk partials per item (sequence b, kv head g, ATTN_CPI_B consecutive chunks), the single-sequence
// phase's numerics (ref_numpy.py:116-129 in chunked form) with a pipelined schedule: the item's K and V tiles were
// issued one item earlier into the other LDS buffer, so after the wait for them the next item's tiles are issued and
// stream in while this item computes; the two chunks' score chains (ascending d) and P.V chains (ascending t) are
// interleaved, with the tile reads a block ahead.  The partials go to global memory and the merge is the next phase
// (no counter: nothing in the item loop waits for a store).
template <int B, class S, class Wait>
__device__ __forceinline__ void phase_attn_b(const Params& p, int layer, S& s, Wait wait) {
  constexpr int CPI = ATTN_CPI_B;
  static_assert(CPI == 2, "the score and P.V loops interleave two chunks");
  const int NKV = p.NKV, NH = p.NH, G = NH / NKV, HD = HDIM, BS = p.BS;
  const int NQKV = (NH + 2 * NKV) * HD;
  const int nitems = p.ibase[p.B];
  const LayerW Lw = layer_w(p, layer);
  const int lane = lane_id(), wave = wave_u();
  // positions from first_new(pos) on are this launch's (the row's own, and in prefill the earlier rows'): patched
  // into the tiles from the QKV rows, not read from the cache
  auto first_new = [&](int pos) { return p.pf ? p.posb[0] : pos; };
  // wave w copies K dim-groups 2w, 2w+1 (lane = position) and the V position-group w (lane = dim, both halves) of
  // every chunk of the item, HBM -> LDS buffer `buf` (global_load_lds, 16 bytes per lane).  The block-table entries
  // they need are read one item ahead (kv_blocks), so issuing the copies waits on nothing.
  struct KvBlocks {
    int k[CPI], v[CPI];                                   // block of the lane's K position, of the wave's V group
  };
  auto kv_blocks = [&](int item) {
    const AttnItem it = attn_item<B, CPI>(p, item);
    const int n = it.pos + 1, fp = first_new(it.pos);
    const int32_t* btab = p.btab + (size_t)it.b * p.nbps;
    KvBlocks r;
#pragma unroll
    for (int ci = 0; ci < CPI; ++ci) {
      const int t0 = (it.cp * CPI + ci) * CHUNK, t = t0 + lane, tb = t0 + wave * 8;
      r.k[ci] = t < n && t < fp ? ld_i(btab + t / BS) : 0;
      r.v[ci] = tb < n && tb < fp ? ld_i(btab + tb / BS) : 0;
    }
    return r;
  };
  auto load_kv = [&](int item, int buf, const KvBlocks& kb) {
    const AttnItem it = attn_item<B, CPI>(p, item);
    const int g = it.g, pos = it.pos, n = pos + 1, nch = (n + CHUNK - 1) / CHUNK, fp = first_new(pos);
#pragma unroll
    for (int ci = 0; ci < CPI; ++ci) {
      const int c = it.cp * CPI + ci;
      if (c < nch) {
        const int t0 = c * CHUNK, len = min(CHUNK, n - t0);
        const int t = t0 + lane;
        if (lane < len && t < fp) {
          const uint16_t* kp = Lw.kc + (((size_t)kb.k[ci] * NKV + g) * (HD / 8)) * BS * 8 + (t % BS) * 8;
#pragma unroll
          for (int jj = 2 * wave; jj < 2 * wave + 2; ++jj)
            __builtin_amdgcn_global_load_lds((const MK_G void*)(kp + (size_t)jj * BS * 8),
                                             (__attribute__((address_space(3))) void*)&s.a.kt[buf][ci][jj][0], 16, 0, 0);
        }
        const int tb = t0 + wave * 8;                     // 8 positions per 16-byte load
        if (tb < t0 + len && tb < fp) {
          const uint16_t* vp = Lw.vc + ((size_t)kb.v[ci] * NKV + g) * HD * BS + tb % BS;
          const int lo = lane_id() * BS;                  // dim lane, lane + 64 (recomputed per load)
          __builtin_amdgcn_global_load_lds((const MK_G void*)(vp + lo),
                                           (__attribute__((address_space(3))) void*)&s.a.vt[buf][ci][wave][0][0], 16, 0, 0);
          __builtin_amdgcn_global_load_lds((const MK_G void*)(vp + lo + 64 * BS),
                                           (__attribute__((address_space(3))) void*)&s.a.vt[buf][ci][wave][1][0], 16, 0, 0);
        }
      }
    }
  };
  const float qn0 = bf2f(ld_u16(Lw.qn + lane)), qn1 = bf2f(ld_u16(Lw.qn + lane + 64));
  const float kn0 = bf2f(ld_u16(Lw.kn + lane)), kn1 = bf2f(ld_u16(Lw.kn + lane + 64));
  if ((int)blockIdx.x < nitems) load_kv(blockIdx.x, 0, kv_blocks(blockIdx.x));
  if (!wait()) return;
  int k = 0;
  for (int item = blockIdx.x; item < nitems; item += p.nwg, ++k) {
    const int buf = k & 1;
    const AttnItem it = attn_item<B, CPI>(p, item);
    const int g = it.g, pos = it.pos, n = pos + 1, nch = (n + CHUNK - 1) / CHUNK;
    const int c0 = it.cp * CPI, nc = min(CPI, nch - c0);   // chunks c0 .. c0 + nc - 1
    const int32_t* btab = p.btab + (size_t)it.b * p.nbps;
    const float* qkv = p.qkv + (size_t)it.b * NQKV;
    float* apart = p.apart + (size_t)it.b * NH * MAX_CHUNKS * PART;
    // this launch's positions in the item's chunks: [qlo, qhi] (decode: pos alone, in the item of the last chunk)
    const int qlo = max(first_new(pos), c0 * CHUNK), qhi = min(pos, (c0 + nc) * CHUNK - 1);
    const float rc = ld_f(p.rope_cos + (size_t)pos * (HD / 2) + lane), rs = ld_f(p.rope_sin + (size_t)pos * (HD / 2) + lane);
    const bool more = item + p.nwg < nitems;
    KvBlocks nkb;                                         // the next item's blocks, read with this item's inputs
    if (more) nkb = kv_blocks(item + p.nwg);
    // wave j: head g*G + j, its roped q in registers (dims lane, lane + 64), broadcast with v_readlane below
    const int j = wave;
    float q0 = 0.0f, q1 = 0.0f;
    if (j < G) {
      const float* src = qkv + (size_t)(g * G + j) * HD;
      float a0 = ld_ag(src + lane), a1 = ld_ag(src + lane + 64);
      if (p.qk_norm) qk_norm(a0, a1, qn0, qn1, p.eps);
      q0 = bfr(bfr(a0 * rc) + bfr(-a1 * rs));
      q1 = bfr(bfr(a1 * rc) + bfr(a0 * rs));
    }
    // k (normed, roped at its position) and v of the launch's positions: position q from QKV row it.b - (pos - q);
    // wave NWAVE-1-w takes positions qlo + w and qlo + w + NWAVE (a launch has <= 2*NWAVE rows)
    float kn[2][2], vn[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int q = qlo + (NWAVE - 1 - wave) + u * NWAVE;
      if (q <= qhi) {
        const float* row = p.qkv + (size_t)(it.b - (pos - q)) * NQKV;
        float a0 = ld_ag(row + (size_t)(NH + g) * HD + lane), a1 = ld_ag(row + (size_t)(NH + g) * HD + lane + 64);
        vn[u][0] = ld_ag(row + (size_t)(NH + NKV + g) * HD + lane);
        vn[u][1] = ld_ag(row + (size_t)(NH + NKV + g) * HD + lane + 64);
        float cq = rc, sq = rs;
        if (q != pos) {
          cq = ld_f(p.rope_cos + (size_t)q * (HD / 2) + lane);
          sq = ld_f(p.rope_sin + (size_t)q * (HD / 2) + lane);
        }
        if (p.qk_norm) qk_norm(a0, a1, kn0, kn1, p.eps);
        kn[u][0] = bfr(bfr(a0 * cq) + bfr(-a1 * sq));
        kn[u][1] = bfr(bfr(a1 * cq) + bfr(a0 * sq));
      }
    }
    __builtin_amdgcn_s_waitcnt(0);                        // this item's tiles (and this wave's loads) have landed
    __syncthreads();                                      // ... in every wave; the other buffer is free
#pragma unroll
    for (int u = 0; u < 2; ++u) {                         // the new positions' bf16 k, v into the tiles
      const int q = qlo + (NWAVE - 1 - wave) + u * NWAVE;
      if (q <= qhi) {
        const int ci = q / CHUNK - c0, tn = q % CHUNK;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int d = lane + 64 * h;
          ((uint16_t*)&s.a.kt[buf][ci][d / 8][tn])[d % 8] = f2bf(kn[u][h]);
          ((uint16_t*)&s.a.vt[buf][ci][tn / 8][h][lane])[tn % 8] = f2bf(vn[u][h]);
        }
        if (q == pos) {                                   // paged append (:121): K [blk][NKV][HD/8][BS][8], V [blk][NKV][HD][BS]
          const int blk = ld_i(btab + pos / BS), off = pos % BS;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int d = lane + 64 * h;
            st_u16(Lw.kc + ((((size_t)blk * NKV + g) * (HD / 8) + d / 8) * BS + off) * 8 + d % 8, f2bf(kn[u][h]));
            st_u16(Lw.vc + (((size_t)blk * NKV + g) * HD + d) * BS + off, f2bf(vn[u][h]));
          }
        }
      }
    }
    __syncthreads();
    if (more) load_kv(item + p.nwg, buf ^ 1, nkb);
    if (j < G) {
      // scores (:126), lane = position: both chunks' chains over ascending d, each q value (an LDS broadcast read)
      // feeding both; the K and q reads run a block of GB dim groups ahead.  With one chunk the second chain reads
      // stale LDS, unused.
      constexpr int GB = 2, NB = HDIM / 8 / GB;
      float* qw = s.a.qb[j];
      qw[lane] = q0;
      qw[lane + 64] = q1;
      float acc0 = 0.0f, acc1 = 0.0f;
      u32x4 kA[2][GB], kB[2][GB];
      mk_f32x4 qA[GB][2], qB[GB][2];
      auto ldk = [&](u32x4(&kk)[2][GB], mk_f32x4(&qq)[GB][2], int blk) {
#pragma unroll
        for (int u = 0; u < GB; ++u) {
          kk[0][u] = s.a.kt[buf][0][blk * GB + u][lane];
          kk[1][u] = s.a.kt[buf][1][blk * GB + u][lane];
          qq[u][0] = *(const mk_f32x4*)(qw + 8 * (blk * GB + u));
          qq[u][1] = *(const mk_f32x4*)(qw + 8 * (blk * GB + u) + 4);
        }
      };
      auto fmk = [&](const u32x4(&kk)[2][GB], const mk_f32x4(&qq)[GB][2]) {
#pragma unroll
        for (int u = 0; u < GB; ++u) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float qa = qq[u][e >> 1][2 * (e & 1)], qb = qq[u][e >> 1][2 * (e & 1) + 1];   // dims d, d + 1
            acc0 = __builtin_fmaf(qa, bf_lo(kk[0][u][e]), acc0);
            acc1 = __builtin_fmaf(qa, bf_lo(kk[1][u][e]), acc1);
            acc0 = __builtin_fmaf(qb, bf_hi(kk[0][u][e]), acc0);
            acc1 = __builtin_fmaf(qb, bf_hi(kk[1][u][e]), acc1);
          }
        }
      };
      ldk(kA, qA, 0);
#pragma unroll
      for (int blk = 0; blk < NB; blk += 2) {
        ldk(kB, qB, blk + 1);
        fmk(kA, qA);
        if (blk + 2 < NB) ldk(kA, qA, blk + 2);
        fmk(kB, qB);
      }
      const int len0 = min(CHUNK, n - c0 * CHUNK), len1 = nc > 1 ? min(CHUNK, n - (c0 + 1) * CHUNK) : 0;
      const float sc0 = lane < len0 ? acc0 * p.attn_scale : -__builtin_huge_valf();
      const float sc1 = lane < len1 ? acc1 * p.attn_scale : -__builtin_huge_valf();
      const float m0 = wave_max(sc0), m1 = wave_max(sc1);
      const float pr0 = lane < len0 ? expf_mk(sc0 - m0) : 0.0f;
      const float pr1 = lane < len1 ? expf_mk(sc1 - m1) : 0.0f;
      float* pw0 = s.a.pb[j][0];
      float* pw1 = s.a.pb[j][1];
      pw0[lane] = pr0;                                    // read back as LDS broadcasts by the P.V chains
      pw1[lane] = pr1;
      // V (:127-128), lanes = dims (lane, lane + 64): a = sum_t p_t v_t[d] and l = sum_t p_t over ascending t
      float a[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}}, l[2] = {0.0f, 0.0f};
      auto vat = [](const u32x4& w, int e) { return (e & 1) ? bf_hi(w[e >> 1]) : bf_lo(w[e >> 1]); };
      if (len1 == CHUNK) {                                // two full chunks: both chains together, reads ahead
        u32x4 vA[4], vB[4];
        mk_f32x4 pA[4], pB[4];                               // positions 8 hb .. + 7 of chunk 0 (0, 1), chunk 1 (2, 3)
        auto ldv = [&](u32x4(&v)[4], mk_f32x4(&pp)[4], int hb) {
          v[0] = s.a.vt[buf][0][hb][0][lane];
          v[1] = s.a.vt[buf][0][hb][1][lane];
          v[2] = s.a.vt[buf][1][hb][0][lane];
          v[3] = s.a.vt[buf][1][hb][1][lane];
          pp[0] = *(const mk_f32x4*)(pw0 + 8 * hb);
          pp[1] = *(const mk_f32x4*)(pw0 + 8 * hb + 4);
          pp[2] = *(const mk_f32x4*)(pw1 + 8 * hb);
          pp[3] = *(const mk_f32x4*)(pw1 + 8 * hb + 4);
        };
        auto fmv = [&](const u32x4(&v)[4], const mk_f32x4(&pp)[4]) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float p0 = pp[e >> 2][e & 3], p1 = pp[2 + (e >> 2)][e & 3];
            a[0][0] = __builtin_fmaf(p0, vat(v[0], e), a[0][0]);
            a[0][1] = __builtin_fmaf(p0, vat(v[1], e), a[0][1]);
            l[0] = l[0] + p0;
            a[1][0] = __builtin_fmaf(p1, vat(v[2], e), a[1][0]);
            a[1][1] = __builtin_fmaf(p1, vat(v[3], e), a[1][1]);
            l[1] = l[1] + p1;
          }
        };
        ldv(vA, pA, 0);
#pragma unroll
        for (int hb = 0; hb < CHUNK / 8; hb += 2) {
          ldv(vB, pB, hb + 1);
          fmv(vA, pA);
          if (hb + 2 < CHUNK / 8) ldv(vA, pA, hb + 2);
          fmv(vB, pB);
        }
      } else {                                            // a partial last chunk: one chunk at a time
#pragma unroll
        for (int ci = 0; ci < CPI; ++ci) {
          const int len = ci == 0 ? len0 : len1;
          const float* pwc = ci == 0 ? pw0 : pw1;
          for (int hb = 0; hb < CHUNK / 8 && hb * 8 < len; ++hb) {
            const u32x4 w0 = s.a.vt[buf][ci][hb][0][lane], w1 = s.a.vt[buf][ci][hb][1][lane];
            const mk_f32x4 pl = *(const mk_f32x4*)(pwc + 8 * hb), ph = *(const mk_f32x4*)(pwc + 8 * hb + 4);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              if (hb * 8 + e < len) {
                const float pt = e < 4 ? pl[e] : ph[e - 4];
                a[ci][0] = __builtin_fmaf(pt, vat(w0, e), a[ci][0]);
                a[ci][1] = __builtin_fmaf(pt, vat(w1, e), a[ci][1]);
                l[ci] = l[ci] + pt;
              }
            }
          }
        }
      }
#pragma unroll
      for (int ci = 0; ci < CPI; ++ci) {
        if (ci < nc) {
          float* part = apart + ((size_t)(g * G + j) * MAX_CHUNKS + c0 + ci) * PART;
          st_ag(part + lane, a[ci][0]);
          st_ag(part + lane + 64, a[ci][1]);
          if (lane == 0) { st_ag(part + HD, ci == 0 ? m0 : m1); st_ag(part + HD + 1, l[ci]); }
        }
      }
    }
    if (p.trace && threadIdx.x == 0)                      // slot 2 of the attention phase: chunk partials issued
      *(MK_G uint64_t*)(p.trace + ((size_t)s.phase * p.nwg + blockIdx.x) * 3 + 2) = __builtin_amdgcn_s_memrealtime();
  }
}

// P2b (batched): per (sequence b, head h), one wave: the merge of the head's chunk partials in ascending chunk order
// (M = max m_c, w_c = exp(m_c - M), L = sum w_c l_c, A[d] = sum w_c a_c[d], o = bf16(A / L)), written as the O
// projection's lane-permuted bf16 row, where dims lane and lane + 64 of a head are adjacent (NH*HD a multiple of 512,
// HD = 128): one 4-byte store per lane.  The waves of the grid take the merges in turn across the workgroups.
template <int B, class S, class Wait>
__device__ __forceinline__ void phase_attn_merge_b(const Params& p, S& s, Wait wait) {
  const int NH = p.NH, HD = HDIM, KA = NH * HD;
  const int lane = lane_id(), wave = wave_u();
  if (!wait()) return;
  for (int m = wave * p.nwg + (int)blockIdx.x; m < p.B * NH; m += p.nwg * NWAVE) {
    const int b = m / NH, h = m - b * NH, nch = p.posb[b] / CHUNK + 1;
    const float* part = p.apart + ((size_t)b * NH + h) * MAX_CHUNKS * PART;
    float* wl = s.m.p[wave];
    // lane cc holds chunks cc and cc + 64's (m, l); the chunk weights go through LDS for the ordered sums.  The
    // first MB chunks' a[] are loaded together with (m, l) (they do not depend on the maximum): one round trip.
    constexpr int MB = 18;
    float av0[MB], av1[MB];
    auto load_a = [&](int cb) {
#pragma unroll
      for (int u = 0; u < MB; ++u) {
        const int c = min(cb + u, nch - 1);               // past the last chunk: a repeat, never used
        av0[u] = ld_ag(part + (size_t)c * PART + lane);
        av1[u] = ld_ag(part + (size_t)c * PART + lane + 64);
      }
    };
    float mloc = -__builtin_huge_valf(), lloc = 0.0f, mhi = -__builtin_huge_valf(), lhi = 0.0f;
    if (lane < nch) { mloc = ld_ag(part + (size_t)lane * PART + HD); lloc = ld_ag(part + (size_t)lane * PART + HD + 1); }
    if (lane + 64 < nch) {
      mhi = ld_ag(part + (size_t)(lane + 64) * PART + HD);
      lhi = ld_ag(part + (size_t)(lane + 64) * PART + HD + 1);
    }
    load_a(0);
    const float M = wave_max(fmaxf(mloc, mhi));
    wl[lane] = lane < nch ? expf_mk(mloc - M) : 0.0f;
    wl[64 + lane] = lane + 64 < nch ? expf_mk(mhi - M) : 0.0f;
    wl[MAX_CHUNKS + lane] = lloc;
    wl[MAX_CHUNKS + 64 + lane] = lhi;
    float Ls = 0.0f, A0 = 0.0f, A1 = 0.0f;
    for (int cb = 0; cb < nch; cb += MB) {
      if (cb > 0) load_a(cb);
#pragma unroll
      for (int u = 0; u < MB; ++u)
        if (cb + u < nch) {
          const float wc = wl[cb + u];
          Ls = __builtin_fmaf(wc, wl[MAX_CHUNKS + cb + u], Ls);
          A0 = __builtin_fmaf(wc, av0[u], A0);
          A1 = __builtin_fmaf(wc, av1[u], A1);
        }
    }
    const int st = perm_stored(h * HD + lane, KA);
    st_ag_u32((uint32_t*)(p.o16 + (size_t)b * KA + st), (uint32_t)f2bf(A0 / Ls) | ((uint32_t)f2bf(A1 / Ls) << 16));
  }
}

// P3: O projection + residual per sequence (ref_numpy.py:130)
template <class WR, int B, class S, class Wait>
__device__ __forceinline__ void phase_oproj_b(const Params& p, int layer, S& s, Wait wait) {
  constexpr int KK = WR::K;
  static_assert(B * KK <= S::XCAP, "attention rows exceed the LDS budget");
  const LayerW Lw = layer_w(p, layer);
  const int H = p.H, nb = p.B, nw = p.nwg * NWAVE;
  const bool first = layer == p.l0 && p.do_embed;
  const uint8_t* W = Lw.wo;
  gemv_run_b<WR, 1, B>(
      H, [&](int g, int) -> const uint8_t* { return mrow<WR>(W, g); }, [&](int) { return nb; },
      [&](int, int b) { return (const uint16_t*)(s.v.xs + b * KK); },
      [&](int g, int nv, const float(&v)[1][B]) {
        const int r = res_slot(g, nw);
        lane_store_b<1, B>(v, nv, [&](int, int b, float val, bool ok) {
          st_ag_u16(ok ? p.x16 + (size_t)b * H + g : (uint16_t*)sink_of(p), f2bf(s.v.xres[b][r] + bfr(val)));
        });
      },
      [&]() {
        load_res_rows<B>(p, H, first, s);
        if (!wait()) return false;
        copy_rows_lds(p.o16, nb * KK, s.v.xs);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        return true;
      },
      p.nwg, p.trace, s.phase);
}

// P4: post-attention RMSNorm + router GEMV per sequence (ref_numpy.py:131-134)
template <int KK, int B, class S, class Wait>
__device__ __forceinline__ void phase_router_b(const Params& p, int layer, S& s, Wait wait) {
  using WR = Bf16Row<KK>;                                 // the router stays bf16 in every weight type
  const LayerW Lw = layer_w(p, layer);
  const int E = p.E, nb = p.B;
  const uint8_t* W = Lw.wr;
  gemv_run_b<WR, 1, B>(
      E, [&](int g, int) -> const uint8_t* { return mrow<WR>(W, g); }, [&](int) { return nb; },
      [&](int, int b) { return (const uint16_t*)(s.n.xs + b * KK); },
      [&](int g, int nv, const float(&v)[1][B]) {
        lane_store_b<1, B>(v, nv, [&](int, int b, float val, bool ok) {
          st_ag(ok ? p.logits + (size_t)b * E + g : sink_of(p), bfr(val));
        });
      },
      [&]() {
        if (!wait()) return false;
        build_norm_xb<KK, B>(p, false, Lw.ln2, s);
        return true;
      },
      p.nwg, p.trace, s.phase);
}

// Top-k of every sequence (wave w routes sequences w, w + 8, its logits loads issued together), then the routed
// (sequence, slot) pairs sorted by (expert, sequence) and the distinct experts in ascending order.  The sort: every
// pair sets bit expert * MAX_B + sequence of a bitmap (keys are distinct), one wave turns the words into prefix
// popcounts, and a pair's rank is the prefix of its word plus the set bits below it.  Every workgroup computes the
// same lists from the same logits.
template <int B, int EC, class S>
__device__ __forceinline__ void route_all(const Params& p, S& s) {
  constexpr int PW = (B + NWAVE - 1) / NWAVE;             // sequences per wave
  const int nb = p.B, K = p.TOPK, np = nb * K, lane = lane_id(), wave = wave_u();
  for (int t = threadIdx.x; t < KEY_WORDS; t += NT) s.kbits[t] = 0u;
  RouteLogits<EC> lg[PW];
#pragma unroll
  for (int j = 0; j < PW; ++j)
    if (wave + NWAVE * j < nb) route_load<EC>(p, p.logits + (size_t)(wave + NWAVE * j) * p.E, lg[j]);
#pragma unroll
  for (int j = 0; j < PW; ++j) {
    const int b = wave + NWAVE * j;
    if (b < nb) route_topk_from<EC>(p, lg[j], &s.rids[b][0], &s.rwts[b][0], nullptr);
  }
  __syncthreads();
  int key = 0;
  if ((int)threadIdx.x < np) {
    const int b = threadIdx.x / K, k = threadIdx.x - b * K;
    key = s.rids[b][k] * MAX_B + b;
    atomicOr(&s.kbits[key >> 5], 1u << (key & 31));
  }
  __syncthreads();
  if (wave == 0) {                                         // exclusive prefix popcount of the words, lane by lane
    uint32_t carry = 0;
    for (int w0 = 0; w0 < KEY_WORDS; w0 += 64) {
      const int wd = w0 + lane;
      const uint32_t c = wd < KEY_WORDS ? (uint32_t)__builtin_popcount(s.kbits[wd]) : 0u;
      uint32_t incl = c;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = (uint32_t)__shfl_up((int)incl, d, 64);
        if (lane >= d) incl += o;
      }
      if (wd < KEY_WORDS) s.kpre[wd] = carry + incl - c;
      carry += (uint32_t)__shfl((int)incl, 63, 64);
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < np) {
    const int b = threadIdx.x / K, k = threadIdx.x - b * K;
    const int rank = (int)s.kpre[key >> 5] + __builtin_popcount(s.kbits[key >> 5] & ((1u << (key & 31)) - 1u));
    s.pexp[rank] = s.rids[b][k];
    s.pseq[rank] = b;
    s.pw[rank] = s.rwts[b][k];
    int j = 0;                                            // the pair's place among its sequence's experts
    for (int k2 = 0; k2 < K; ++k2) j += s.rids[b][k2] < s.rids[b][k];
    s.bpair[b][j] = rank;
  }
  __syncthreads();
  if (wave == 0) {                                         // first pair of each expert -> ustart
    int carry = 0;
    for (int c0 = 0; c0 < np; c0 += 64) {
      const int t = c0 + lane;
      const bool head = t < np && (t == 0 || s.pexp[t] != s.pexp[t - 1]);
      const uint64_t m = __ballot(head);
      if (head) {
        const int u = carry + __builtin_popcountll(m & ((1ull << lane) - 1ull));
        s.uexp[u] = s.pexp[t];
        s.ustart[u] = t;
      }
      carry += __builtin_popcountll(m);
    }
    if (lane == 0) {
      s.nexp = carry;
      s.ustart[carry] = np;
    }
  }
  __syncthreads();
}

// P5: routing, then each distinct expert's gate/up rows against the normed rows of the sequences routed to it,
// SiLU*up into that pair's h16 row (ref_numpy.py:135-145)
template <class WR, int B, int EC, class S, class Wait>
__device__ __forceinline__ void phase_expert_up_b(const Params& p, int layer, S& s, Wait wait) {
  constexpr int KK = WR::K;
  const LayerW Lw = layer_w(p, layer);
  const int MI = p.MI, KT = p.TOPK, nb = p.B;
  const uint8_t* W = Lw.w13;
  build_norm_xb<KK, B>(p, false, Lw.ln2, s);              // x is final since the O projection
  if (!wait()) return;
  route_all<B, EC>(p, s);
  if (blockIdx.x == 0) {
    for (int t = threadIdx.x; t < nb * KT; t += NT) {
      const int b = t / KT, k = t - b * KT;
      if (p.dump_ids) st_i(p.dump_ids + ((size_t)layer * nb + b) * KT + k, s.rids[b][k]);
      if (p.dump_wts) st_f(p.dump_wts + ((size_t)layer * nb + b) * KT + k, s.rwts[b][k]);
    }
    if (p.dump_logits)
      for (int t = threadIdx.x; t < nb * p.E; t += NT) st_f(p.dump_logits + (size_t)layer * nb * p.E + t, ld_ag(p.logits + t));
  }
  const int U = s.nexp;
  gemv_run_b<WR, 2, B>(
      U * MI,
      [&](int g, int i) -> const uint8_t* {
        const int u = g / MI, j = g - u * MI;
        return mrow<WR>(W, (size_t)s.uexp[u] * 2 * MI + 2 * j + i);
      },
      [&](int g) { const int u = g / MI; return s.ustart[u + 1] - s.ustart[u]; },
      [&](int g, int b) { return (const uint16_t*)(s.n.xs + s.pseq[s.ustart[g / MI] + b] * KK); },
      [&](int g, int nv, const float(&v)[2][B]) {
        const int u = g / MI, j = g - u * MI, lane = lane_id();
        const float gv = lane_pick<1, B>((const float(&)[1][B])v[0]), uv = lane_pick<1, B>((const float(&)[1][B])v[1]);
        st_ag_u16(lane < nv ? p.h16 + (size_t)(s.ustart[u] + lane) * MI + perm_stored(j, MI) : (uint16_t*)sink_of(p),
                  f2bf(bfr(bfr(silu(bfr(gv))) * bfr(uv))));
      },
      [&]() { return true; }, p.nwg, p.trace, s.phase);
}

// P5 on the matrix cores (handles of batch capacity >= 8, p.mfma): tiles of 16 consecutive gate/up rows of one
// routed expert against the sequences routed to it (at most 16: one MFMA column each, the others zero), D = W X
// through chained v_mfma_f32_16x16x32_bf16 from 0.  Lane l (row l % 16, quad q = l / 16) loads the 16-byte lane slot
// 4s + q of its row in every block, so one block of the tile's 16 rows is 16 loads per lane (16 KB, bf16 512-element
// blocks; an e4m3 row's 1024-element block is the same 16 loads, each slot's codes 0-7 paired with the input's even
// 512-block and codes 8-15 with the odd one, decoded to bf16 exactly); the input operand is the same slot of the
// sequence's normed row in LDS.  The sum's order is therefore: 512-element blocks ascending, 16 steps a block, step s
// giving quad q the elements 4s + q + 64 j (j < 8), each step by the hardware's accumulation rule (the oracle's
// mfma_bf16_k32).  Two register buffers alternate: the next block's loads are issued before this block's MFMAs; past
// the wave's last block the issue reads the wave's sink line, so every issue is the same run of loads.  D's lane holds
// rows 4q .. 4q + 3 of one sequence, two whole gate/up pairs: SiLU * up is formed in the lane.

// codes 8h .. 8h + 7 of a 16-code e4m3 slot as 8 bf16 (exact: every e4m3 value is a bf16 value)
__device__ __forceinline__ mk_bf16x8 e4m3_half_bf16(const u32x4& c, int h) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  u32x4 o;
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const uint32_t w = c[2 * h + d];
    // gfx950's v_cvt_scalef32_pk_bf16_fp8 at scale 1: codes 0, 1 (then 2, 3) of the word to a bf16 pair, low half
    // first; every e4m3 value is a bf16 value, so the conversion is exact
    o[2 * d] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, false));
    o[2 * d + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, true));
  }
  return __builtin_bit_cast(mk_bf16x8, o);
}

// The tile engine: tiles t = gw, gw + nw, ... of the calling wave; tile t's A rows are rowf(t) (the format row of
// the lane's row, l % 16 of the tile), its B columns colf(t, has) (the LDS input row of the lane's column; has = false
// makes the column zero, and the row returned must still be an LDS row of KK elements); epi(t, v) receives D rows 4q .. 4q + 3 of the lane's column (fp8: times each row's scale).  The first
// block's loads are issued before prologue() (which may wait and synchronise the workgroup; every thread calls it
// once); rowf must then not depend on what the prologue waits for.
template <class WR, class RowF, class ColF, class EpiF, class Pro>
__device__ __forceinline__ bool mfma_tiles(const Params& p, int ntile, RowF rowf, ColF colf, EpiF epi, Pro prologue,
                                           int s_phase) {
  constexpr int KK = WR::K;
  constexpr bool F8 = WR::FP8;
  constexpr int NBLK = F8 ? KK / 1024 : KK / 512;
  static_assert(KK % (F8 ? 1024 : 512) == 0 && NBLK >= 1, "the tile path takes whole blocks");
  const int gw = blockIdx.x * NWAVE + wave_u(), nw = p.nwg * NWAVE;
  const int nitem = (gw < ntile ? (ntile - 1 - gw) / nw + 1 : 0) * NBLK;
  const uint8_t* sinkp = (const uint8_t*)sink_of(p);
  // the lane's quad, recomputed at each use (lane_id: no lane-dependent address is held across phases)
  auto issue = [&](int it, u32x4(&R)[16], float& sc) {
    const int q = lane_id() >> 4;
    const bool ok = it < nitem;
    const uint8_t* row = ok ? rowf(gw + (it / NBLK) * nw) : sinkp;
    const uint8_t* base = ok ? row + 1024 * (it % NBLK) + 16 * q : sinkp + 16 * q;
    const int step = ok ? 64 : 0;
    // ordinary (cached) loads: a wave's load of one slot column reads 64 bytes of each of its 16 rows, and the next
    // slot column the other half of the same 128-byte lines; non-temporal loads let those lines go between the two
    // (2.3 GB more fetched per batch-16 fp8 step, 13.75 against 12.99 ms)
#pragma unroll
    for (int i = 0; i < 16; ++i) R[i] = ld16(base + step * i);
    if constexpr (F8) sc = ld_f((const float*)(ok ? row + KK : sinkp));
  };
  mk_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](int it, const u32x4(&R)[16], float sc) {
    const int blk = it % NBLK, t = gw + (it / NBLK) * nw, q = lane_id() >> 4;
    if (blk == 0) acc = mk_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    bool has;
    const uint16_t* xb = colf(t, has) + 8 * q;
    auto xop = [&](int xblk, int i) -> mk_bf16x8 {
      const u32x4 v = *(const u32x4*)(xb + 512 * xblk + 32 * i);
      return __builtin_bit_cast(mk_bf16x8, has ? v : u32x4{0u, 0u, 0u, 0u});
    };
    if constexpr (!F8) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mk_bf16x8, R[i]), xop(blk, i), acc, 0, 0, 0);
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(e4m3_half_bf16(R[i], h), xop(2 * blk + h, i), acc, 0, 0, 0);
    }
    if (blk == NBLK - 1) {
      // the epilogue reads the chain's last MFMA result: the compiler's own wait before that read (s_nop 7, 8 wait
      // states) let 4 of 32 768 values be read before the result was complete (each differing from the finished
      // sum); 18 wait states, fenced against rescheduling, make the read follow the write
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 1" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = F8 ? acc[i] * __shfl(sc, 4 * q + i) : acc[i];   // row 4q + i's scale
      epi(t, v);
    }
  };
  u32x4 R0[16], R1[16];
  float sc0 = 1.0f, sc1 = 1.0f;
  issue(0, R0, sc0);
  if (p.trace && threadIdx.x == 0)
    *(MK_G uint64_t*)(p.trace + ((size_t)s_phase * p.nwg + blockIdx.x) * 3 + 2) = __builtin_amdgcn_s_memrealtime();
  if (!prologue()) return false;
  if (nitem == 0) return true;
  for (int it = 0;;) {
    issue(it + 1, R1, sc1);
    compute(it, R0, sc0);
    if (++it >= nitem) break;
    issue(it + 1, R0, sc0);
    compute(it, R1, sc1);
    if (++it >= nitem) break;
  }
  return true;
}

template <class WR, int B, int EC, class S, class Wait>
__device__ __forceinline__ void phase_expert_up_mfma(const Params& p, int layer, S& s, Wait wait) {
  constexpr int KK = WR::K;
  const LayerW Lw = layer_w(p, layer);
  const int MI = p.MI, KT = p.TOPK, nb = p.B;
  const uint8_t* W = Lw.w13;
  // the normed rows: left in LDS by the router phase (every workgroup normed them there; nothing since wrote s.n)
  if (!wait()) return;
  route_all<B, EC>(p, s);
  if (blockIdx.x == 0) {
    for (int t = threadIdx.x; t < nb * KT; t += NT) {
      const int b = t / KT, k = t - b * KT;
      if (p.dump_ids) st_i(p.dump_ids + ((size_t)layer * nb + b) * KT + k, s.rids[b][k]);
      if (p.dump_wts) st_f(p.dump_wts + ((size_t)layer * nb + b) * KT + k, s.rwts[b][k]);
    }
    if (p.dump_logits)
      for (int t = threadIdx.x; t < nb * p.E; t += NT) st_f(p.dump_logits + (size_t)layer * nb * p.E + t, ld_ag(p.logits + t));
  }
  const int TPE = (2 * MI) / 16;
  mfma_tiles<WR>(
      p, s.nexp * TPE,
      [&](int t) {
        const int u = t / TPE, jt = t - u * TPE, r = lane_id() & 15;
        return mrow<WR>(W, (size_t)s.uexp[u] * 2 * MI + 16 * jt + r);
      },
      [&](int t, bool& has) -> const uint16_t* {         // column r: the expert's r-th routed sequence
        const int u = t / TPE, p0 = s.ustart[u], r = lane_id() & 15;
        has = r < s.ustart[u + 1] - p0;
        return s.n.xs + (size_t)(has ? s.pseq[p0 + r] : 0) * KK;
      },
      [&](int t, const float(&v)[4]) {                    // rows 4q, 4q+1: pair j0; rows 4q+2, 4q+3: pair j0 + 1
        const int u = t / TPE, jt = t - u * TPE, p0 = s.ustart[u], r = lane_id() & 15, q = lane_id() >> 4;
        const bool has = r < s.ustart[u + 1] - p0;
        const int j0 = 8 * jt + 2 * q;
        const float h0 = bfr(bfr(silu(bfr(v[0]))) * bfr(v[1]));
        const float h1 = bfr(bfr(silu(bfr(v[2]))) * bfr(v[3]));
        // h in the stored order of the down rows it meets (fp8 rows: blocks of 1024), the order the matrix-core
        // down tiles chain over
        uint16_t* hrow = p.h16 + (size_t)(p0 + r) * MI;
        const int s0 = WR::FP8 ? perm_stored8(j0, MI) : perm_stored(j0, MI);
        const int s1 = WR::FP8 ? perm_stored8(j0 + 1, MI) : perm_stored(j0 + 1, MI);
        st_ag_u16(has ? hrow + s0 : (uint16_t*)sink_of(p), f2bf(h0));
        st_ag_u16(has ? hrow + s1 : (uint16_t*)sink_of(p), f2bf(h1));
      },
      [&]() { return true; }, s.phase);
}

// The split form for the dense projections, whose few tiles would leave most waves idle as whole-row chains: tile t
// belongs to workgroup t % nwg as its local tile t / nwg; local item j (tile j / NBLK, block j % NBLK) goes to wave
// j % NWAVE in round j / NWAVE.  Each item runs its block's MFMA chain from zero; the NBLK partial tiles meet in LDS
// and the wave of block 0 adds them as a pairwise tree ((P0 + P1) + (P2 + P3)) ..., scales (fp8) and hands the
// lane's four D rows to epi(t, v).  Round 0's loads are issued before prologue(), each later round's one round ahead.
template <class WR, class S, class RowF, class ColF, class EpiF, class Pro>
__device__ __forceinline__ bool mfma_tiles_split(const Params& p, S& s, int ntile, RowF rowf, ColF colf, EpiF epi,
                                                 Pro prologue) {
  constexpr int KK = WR::K;
  constexpr bool F8 = WR::FP8;
  constexpr int NBLK = F8 ? KK / 1024 : KK / 512;
  static_assert(KK % (F8 ? 1024 : 512) == 0 && NBLK >= 1 && NWAVE % NBLK == 0, "a round holds whole tiles");
  static_assert(sizeof(s.v.xres) + sizeof(s.v.acc) >= sizeof(float) * NWAVE * 256 &&
                    offsetof(S, v.acc) == offsetof(S, v.xres) + sizeof(s.v.xres),
                "the partial tiles live in the residual and combine slots");
  float* part = &s.v.xres[0][0];                          // [wave][lane][4]
  const int w = wave_u(), wg = blockIdx.x, nwg = p.nwg;
  const int nit = (wg < ntile ? (ntile - 1 - wg) / nwg + 1 : 0) * NBLK;
  const int nround = (nit + NWAVE - 1) / NWAVE;
  auto tile_of = [&](int j) { return wg + (j / NBLK) * nwg; };
  auto issue = [&](int j, u32x4(&R)[16], float& sc) {    // j < nit
    const int q = lane_id() >> 4;
    const uint8_t* row = rowf(tile_of(j));
    const uint8_t* base = row + 1024 * (j % NBLK) + 16 * q;
#pragma unroll
    for (int i = 0; i < 16; ++i) R[i] = ld16(base + 64 * i);
    if constexpr (F8) sc = ld_f((const float*)(row + KK));
  };
  auto round = [&](int r, const u32x4(&Rc)[16], float scc, u32x4(&Rn)[16], float& scn) {
    const int j = r * NWAVE + w, lane = lane_id(), q = lane >> 4;
    if (j + NWAVE < nit) issue(j + NWAVE, Rn, scn);
    if (j < nit) {
      const int blk = j % NBLK;
      bool has;
      const uint16_t* xb = colf(tile_of(j), has) + 8 * q;
      auto xop = [&](int xblk, int i) -> mk_bf16x8 {
        const u32x4 v = *(const u32x4*)(xb + 512 * xblk + 32 * i);
        return __builtin_bit_cast(mk_bf16x8, has ? v : u32x4{0u, 0u, 0u, 0u});
      };
      mk_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
      if constexpr (!F8) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mk_bf16x8, Rc[i]), xop(blk, i), acc, 0, 0, 0);
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(e4m3_half_bf16(Rc[i], h), xop(2 * blk + h, i), acc, 0, 0, 0);
      }
      // the chain's last result is read by VALU next: the wait states the compiler's own s_nop 7 leaves were found
      // too few for the gate/up tiles (4 of 32 768 values read early); 18, fenced against rescheduling
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 1" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      *(mk_f32x4*)(part + 4 * (w * 64 + lane)) = acc;
    }
    __syncthreads();
    if (j < nit && j % NBLK == 0) {
      float t[NBLK][4];
#pragma unroll
      for (int k = 0; k < NBLK; ++k) {
        const mk_f32x4 v = *(const mk_f32x4*)(part + 4 * ((w + k) * 64 + lane));
#pragma unroll
        for (int i = 0; i < 4; ++i) t[k][i] = v[i];
      }
#pragma unroll
      for (int width = 1; width < NBLK; width *= 2)
#pragma unroll
        for (int k = 0; k + width < NBLK; k += 2 * width)
#pragma unroll
          for (int i = 0; i < 4; ++i) t[k][i] = t[k][i] + t[k + width][i];
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = F8 ? t[0][i] * __shfl(scc, 4 * q + i) : t[0][i];   // row 4q + i's scale
      epi(tile_of(j), v);
    }
    __syncthreads();                                      // the partial slots are the next round's
  };
  u32x4 R0[16], R1[16];
  float sc0 = 1.0f, sc1 = 1.0f;
  if (w < nit) issue(w, R0, sc0);
  if (p.trace && threadIdx.x == 0)
    *(MK_G uint64_t*)(p.trace + ((size_t)s.phase * p.nwg + blockIdx.x) * 3 + 2) = __builtin_amdgcn_s_memrealtime();
  if (!prologue()) return false;
  for (int r = 0; r < nround;) {
    round(r, R0, sc0, R1, sc1);
    if (++r >= nround) break;
    round(r, R1, sc1, R0, sc0);
    ++r;
  }
  return true;
}

// P1 on the matrix cores (p.mfma): tiles of 16 QKV rows against every sequence's normed row (the columns), split by
// block; the first blocks issued before the wait
template <class WR, int B, class S, class Wait>
__device__ __forceinline__ void phase_qkv_mfma(const Params& p, int layer, S& s, Wait wait) {
  constexpr int KK = WR::K;
  const LayerW Lw = layer_w(p, layer);
  const bool first = layer == p.l0 && p.do_embed;
  const int rows = p.nqkv, nb = p.B;
  const uint8_t* W = Lw.wqkv;
  mfma_tiles_split<WR>(
      p, s, rows / 16, [&](int t) { return mrow<WR>(W, (size_t)16 * t + (lane_id() & 15)); },
      [&](int, bool& has) -> const uint16_t* {
        const int r = lane_id() & 15;
        has = r < nb;
        return s.n.xs + (size_t)(has ? r : 0) * KK;
      },
      [&](int t, const float(&v)[4]) {
        const int r = lane_id() & 15, q = lane_id() >> 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 16 * t + 4 * q + i;
          st_ag(r < nb ? p.qkv + (size_t)r * rows + row : sink_of(p), bfr(v[i]));
        }
      },
      [&]() {
        if (!wait()) return false;
        build_norm_xb<KK, B>(p, first, Lw.ln1, s);
        if (blockIdx.x == 0) {
          if (p.dump_x && layer > p.l0)
            for (int i = threadIdx.x; i < nb * KK; i += NT)
              st_f(p.dump_x + (size_t)(layer - 1) * nb * KK + i, bf2f(s.n.xr[i]));
          if (layer == p.l0 && p.do_head && (int)threadIdx.x < nb)
            __hip_atomic_store(p.amax + 32 * threadIdx.x, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return true;
      });
}

// P3 on the matrix cores (p.mfma): tiles of 16 output rows of the O projection against every sequence's attention
// output (copied into LDS after the wait), split by block, plus the residual read per (row, sequence)
template <class WR, int B, class S, class Wait>
__device__ __forceinline__ void phase_oproj_mfma(const Params& p, int layer, S& s, Wait wait) {
  constexpr int KK = WR::K;
  static_assert(B * KK <= S::XCAP, "attention rows exceed the LDS budget");
  const LayerW Lw = layer_w(p, layer);
  const int H = p.H, nb = p.B;
  const bool first = layer == p.l0 && p.do_embed;
  const uint8_t* W = Lw.wo;
  mfma_tiles_split<WR>(
      p, s, H / 16, [&](int t) { return mrow<WR>(W, (size_t)16 * t + (lane_id() & 15)); },
      [&](int, bool& has) -> const uint16_t* {
        const int r = lane_id() & 15;
        has = r < nb;
        return s.v.xs + (size_t)(has ? r : 0) * KK;
      },
      [&](int t, const float(&v)[4]) {
        const int r = lane_id() & 15, q = lane_id() >> 4;
        const int b = r < nb ? r : 0;
        const int tok = first ? token_of_b(p, b) : 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int g = 16 * t + 4 * q + i;
          const float xres = first ? bf2f(ld_u16(p.embed + (size_t)tok * H + g)) : bf2f(ld_ag_u16(p.x16 + (size_t)b * H + g));
          st_ag_u16(r < nb ? p.x16 + (size_t)b * H + g : (uint16_t*)sink_of(p), f2bf(xres + bfr(v[i])));
        }
      },
      [&]() {
        if (!wait()) return false;
        // tile t is workgroup t % nwg's: with H / 16 tiles on more workgroups, the rest have none and copy nothing
        if ((int)blockIdx.x < H / 16) copy_rows_lds(p.o16, nb * KK, s.v.xs);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        return true;
      });
}

// P4 on the matrix cores (p.mfma): tiles of 16 experts' router rows (bf16) against every sequence's post-attention
// normed row, split by block as the dense projections (E/16 tiles: a few workgroups).  Every workgroup norms the rows
// in its prologue and keeps them in LDS for the gate/up phase.
template <int KK, int B, int EC, class S, class Wait>
__device__ __forceinline__ void phase_router_mfma(const Params& p, int layer, S& s, Wait wait) {
  using WR = Bf16Row<KK>;                                 // the router stays bf16 in every weight type
  static_assert(EC % 16 == 0, "whole router tiles");
  const LayerW Lw = layer_w(p, layer);
  const int nb = p.B;
  mfma_tiles_split<WR>(
      p, s, EC / 16, [&](int t) { return mrow<WR>(Lw.wr, (size_t)16 * t + (lane_id() & 15)); },
      [&](int, bool& has) -> const uint16_t* {
        const int r = lane_id() & 15;
        has = r < nb;
        return s.n.xs + (size_t)(has ? r : 0) * KK;
      },
      [&](int t, const float(&v)[4]) {
        const int r = lane_id() & 15, q = lane_id() >> 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) st_ag(r < nb ? p.logits + (size_t)r * EC + 16 * t + 4 * q + i : sink_of(p), bfr(v[i]));
      },
      [&]() {
        if (!wait()) return false;
        build_norm_xb<KK, B>(p, false, Lw.ln2, s);
        return true;
      });
}

// P6: expert down, routing weight, combine per sequence in ascending expert id, residual (ref_numpy.py:146-148).
// Each wave owns output rows; for its row it streams the rows of every distinct expert (D at a time, the next
// batch in flight while the current one is reduced) and dots each with the h rows of that expert's pairs.  The
// pairs' h rows are staged in LDS in passes of whole experts that fit; lane b carries sequence b's combine chain,
// kept in LDS between batches and passes.  Every batch issue is the same run of loads (a batch short of D experts
// reloads its last one; after a row's last batch the issue reloads it: HBM re-fetches, the rows being streamed
// non-temporally) and the outputs are stored after the last
// pass, so the wait before a batch's dots counts exactly the loads issued after it.
template <class WR, int B, class S, class Wait>
__device__ __forceinline__ void phase_expert_down_b(const Params& p, int layer, S& s, Wait wait) {
  constexpr int KK = WR::K;
  constexpr int PCAP = S::XCAP / KK;                      // pairs per pass
  static_assert(PCAP >= MAX_B, "one expert's pairs must fit a pass");
  constexpr int DE = WR::REGS <= 7 ? 8 : WR::REGS <= 13 ? 4 : 2;
  using Regs = typename WR::Regs;
  const LayerW Lw = layer_w(p, layer);
  const int H = p.H, nb = p.B, nw = p.nwg * NWAVE, lane = lane_id();
  const int gw = blockIdx.x * NWAVE + wave_u();
  const int U = s.nexp;                                   // routing kept from P5
  const uint8_t* W = Lw.w2;
  const int nrw = gw < H ? (H - 1 - gw) / nw + 1 : 0;    // output rows of this wave
  Regs R[2][DE];
  auto issue = [&](Regs(&Rb)[DE], int g, int ub, int u1) {
#pragma unroll
    for (int d = 0; d < DE; ++d) {
      const int u = ub + d < u1 ? ub + d : u1 - 1;
      WR::load(Rb[d], mrow<WR>(W, (size_t)s.uexp[u] * H + g), lane);
    }
  };
  int u0 = 0, u1 = 0;
  auto pass_end = [&](int a) {
    int e = a + 1;
    while (e < U && s.ustart[e + 1] - s.ustart[a] <= PCAP) ++e;
    return e;
  };
  u1 = U > 0 ? pass_end(0) : 0;
  if (nrw > 0 && U > 0) issue(R[0], gw, 0, u1);           // the first batch streams during the wait
  if (p.trace && threadIdx.x == 0)
    *(MK_G uint64_t*)(p.trace + ((size_t)s.phase * p.nwg + blockIdx.x) * 3 + 2) = __builtin_amdgcn_s_memrealtime();
  load_res_rows<B>(p, H, false, s);
  if (!wait()) return;
  bool first_pass = true;
  while (u0 < U) {
    const int p0 = s.ustart[u0];
    const int nbt = (u1 - u0 + DE - 1) / DE, T = nrw * nbt;
    __syncthreads();                                      // the previous pass is done with s.v.xs
    copy_rows_lds(p.h16 + (size_t)p0 * KK, (s.ustart[u1] - p0) * KK, s.v.xs);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    float acc = 0.0f;
    auto compute = [&](Regs(&Rb)[DE], int t) {
      const int g = gw + (t / nbt) * nw, ub = u0 + (t % nbt) * DE, r = res_slot(g, nw);
      if (t % nbt == 0) acc = (!first_pass && lane < nb) ? s.v.acc[lane][r] : 0.0f;
#pragma unroll
      for (int d = 0; d < DE; ++d) settle(Rb[d]);
#pragma unroll
      for (int d = 0; d < DE; ++d)
        if (ub + d < u1)
          for (int pp = s.ustart[ub + d]; pp < s.ustart[ub + d + 1]; ++pp) {
            const float y = bfr(bfr(WR::dot(Rb[d], s.v.xs + (pp - p0) * KK, lane)) * s.pw[pp]);
            if (lane == s.pseq[pp]) acc = bfr(acc + y);
          }
      if (t % nbt == nbt - 1 && lane < nb) s.v.acc[lane][r] = acc;
    };
    auto batch_g = [&](int t) { return gw + (t / nbt) * nw; };
    auto batch_u = [&](int t) { return u0 + (t % nbt) * DE; };
    auto clamp_t = [&](int t) { return t < T ? t : T - 1; };
    if (T > 0) {                                          // a buffer is refilled right after its dots
      if (!first_pass) issue(R[0], batch_g(0), batch_u(0), u1);
      issue(R[1], batch_g(clamp_t(1)), batch_u(clamp_t(1)), u1);
      for (int t = 0;; t += 2) {
        compute(R[0], t);
        if (t + 1 >= T) break;
        issue(R[0], batch_g(clamp_t(t + 2)), batch_u(clamp_t(t + 2)), u1);
        compute(R[1], t + 1);
        if (t + 2 >= T) break;
        issue(R[1], batch_g(clamp_t(t + 3)), batch_u(clamp_t(t + 3)), u1);
      }
    }
    first_pass = false;
    u0 = u1;
    if (u0 < U) u1 = pass_end(u0);
  }
  for (int g = gw; g < H; g += nw)                        // residual + combine (no expert, never with TOPK >= 1:
    if (lane < nb) {                                      // the residual alone)
      const int r = res_slot(g, nw);
      st_ag_u16(p.x16 + (size_t)lane * H + g, f2bf(U > 0 ? s.v.xres[lane][r] + s.v.acc[lane][r] : s.v.xres[lane][r]));
    }
}

// 8 e4m3 codes (two words) as 8 bf16 values, exactly (e4m3_half_bf16 on the low half of a 4-word vector)
__device__ __forceinline__ mk_bf16x8 e4m3_8_bf16(const u32x2& c) { return e4m3_half_bf16(u32x4{c[0], c[1], 0u, 0u}, 0); }
__device__ __forceinline__ u32x2 ld8(const void* p) { return *(const MK_G u32x2*)p; }

// P6 on the matrix cores (p.mfma): tiles of 16 down rows of one expert against its routed pairs' h rows (the
// columns), chained from zero over the rows' stored order in 32-element steps: per lane and step 16 bytes of a bf16
// row or 8 bytes of an fp8 row (whose pairs' h rows the gate/up tiles store in the fp8 order).  Every (pair, row)
// value y = bfr(bfr(d) * weight) goes to p.ys; the combine phase adds them per sequence in ascending expert order.
// The U * H/16 tiles, expert-major, are cut into nwg contiguous ranges, one per workgroup: the workgroup stages the
// h rows of its range's experts in LDS (as many experts at a time as fit) and its waves take the range's tiles
// round-robin, each tile in chunks of 8 steps (256 elements) streamed through a ring of three (two in flight while
// one is chained).  The first chunks are issued before the wait.
template <class WR, int B, class S, class Wait>
__device__ __forceinline__ void phase_expert_down_mfma(const Params& p, int layer, S& s, Wait wait) {
  constexpr int KK = WR::K;
  constexpr bool F8 = WR::FP8;
  constexpr int NC = KK / 256;
  static_assert(KK % 256 == 0, "down rows are whole chunks of 256");
  static_assert(B * KK <= S::XCAP, "one expert's h rows must fit the LDS rows");
  using Chunk = typename std::conditional<F8, u32x2, u32x4>::type;
  const LayerW Lw = layer_w(p, layer);
  const int H = p.H, HT = H / 16, U = s.nexp, w = wave_u(), wg = blockIdx.x, nwg = p.nwg;
  const int T = U * HT;
  const int ta = (int)((int64_t)T * wg / nwg), tb = (int)((int64_t)T * (wg + 1) / nwg);
  const uint8_t* W = Lw.w2;
  // a group: experts [u, ue] of the range whose pairs fit the LDS rows together (at least one expert)
  auto group_end = [&](int u, int ulast) {
    int ue = u;
    while (ue < ulast && (s.ustart[ue + 2] - s.ustart[u]) * KK <= S::XCAP) ++ue;
    return ue;
  };
  int u = ta < tb ? ta / HT : 0;
  const int ulast = ta < tb ? (tb - 1) / HT : -1;
  int ue = u <= ulast ? group_end(u, ulast) : -1;
  int g0 = 0, nit = 0;
  auto set_group = [&]() {
    g0 = ta > u * HT ? ta : u * HT;
    const int g1 = tb < (ue + 1) * HT ? tb : (ue + 1) * HT;
    nit = (g0 + w < g1 ? (g1 - 1 - g0 - w) / NWAVE + 1 : 0) * NC;
  };
  auto tile_of = [&](int it) { return g0 + w + (it / NC) * NWAVE; };
  auto issue = [&](int it, Chunk(&R)[8], float& sc) {    // item it < nit: chunk it % NC of tile tile_of(it)
    const int t = tile_of(it), c = it % NC, ut = t / HT, lane = lane_id(), q = lane >> 4;
    const uint8_t* row = mrow<WR>(W, (size_t)s.uexp[ut] * H + 16 * (t - ut * HT) + (lane & 15));
    if constexpr (F8) {
#pragma unroll
      for (int i = 0; i < 8; ++i) R[i] = ld8(row + 256 * c + 32 * i + 8 * q);
      sc = ld_f((const float*)(row + KK));
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) R[i] = ld16(row + 2 * (256 * c + 32 * i + 8 * q));
    }
  };
  mk_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  auto compute = [&](int it, const Chunk(&R)[8], float sc) {
    const int t = tile_of(it), c = it % NC, ut = t / HT, lane = lane_id(), q = lane >> 4, r = lane & 15;
    const int p0 = s.ustart[ut], np = s.ustart[ut + 1] - p0;
    const bool has = r < np;                              // column r: the expert's r-th pair
    const uint16_t* xb = s.v.xs + (size_t)(has ? p0 - s.ustart[u] + r : 0) * KK + 256 * c + 8 * q;
    if (c == 0) acc = mk_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const u32x4 xv = *(const u32x4*)(xb + 32 * i);
      const mk_bf16x8 bv = __builtin_bit_cast(mk_bf16x8, has ? xv : u32x4{0u, 0u, 0u, 0u});
      mk_bf16x8 av;
      if constexpr (F8) av = e4m3_8_bf16(R[i]);
      else av = __builtin_bit_cast(mk_bf16x8, R[i]);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
    }
    if (c == NC - 1) {
      // the chain's last result read by VALU: 18 wait states, fenced (the compiler's s_nop 7 was found too few)
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 1" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      const float pw = has ? s.pw[p0 + r] : 0.0f;
      const int rt = t - ut * HT;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = F8 ? acc[i] * __shfl(sc, 4 * q + i) : acc[i];   // row 4q + i's scale
        st_ag_u16(has ? p.ys + (size_t)(p0 + r) * H + 16 * rt + 4 * q + i : (uint16_t*)sink_of(p), f2bf(bfr(bfr(v) * pw)));
      }
    }
  };
  Chunk R0[8], R1[8], R2[8];
  float c0 = 1.0f, c1 = 1.0f, c2 = 1.0f;
  if (u <= ulast) {
    set_group();
    if (nit > 0) issue(0, R0, c0);
    if (nit > 1) issue(1, R1, c1);
  }
  if (p.trace && threadIdx.x == 0)
    *(MK_G uint64_t*)(p.trace + ((size_t)s.phase * p.nwg + blockIdx.x) * 3 + 2) = __builtin_amdgcn_s_memrealtime();
  if (!wait()) return;
  for (bool first = true; u <= ulast; first = false) {
    if (!first) {
      set_group();
      if (nit > 0) issue(0, R0, c0);
      if (nit > 1) issue(1, R1, c1);
    }
    const int pb = s.ustart[u];
    __syncthreads();                                      // the previous group is done with the LDS rows
    copy_rows_lds(p.h16 + (size_t)pb * KK, (s.ustart[ue + 1] - pb) * KK, s.v.xs);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int it = 0; it < nit; it += 3) {
      if (it + 2 < nit) issue(it + 2, R2, c2);
      compute(it, R0, c0);
      if (it + 1 >= nit) break;
      if (it + 3 < nit) issue(it + 3, R0, c0);
      compute(it + 1, R1, c1);
      if (it + 2 >= nit) break;
      if (it + 4 < nit) issue(it + 4, R1, c1);
      compute(it + 2, R2, c2);
    }
    u = ue + 1;
    if (u <= ulast) ue = group_end(u, ulast);
  }
}

// P7 (p.mfma): per (sequence, row) the weighted expert outputs of P6 added in ascending expert order, then the
// residual (ref_numpy.py:146-148); workgroup j takes rows [H j / nwg, H (j + 1) / nwg) of every sequence, each
// thread one (sequence, row) with its TOPK values loaded together
template <int B, class S, class Wait>
__device__ __forceinline__ void phase_combine_mfma(const Params& p, S& s, Wait wait) {
  const int H = p.H, nb = p.B, K = p.TOPK, wg = blockIdx.x, nwg = p.nwg;
  const int g0 = (int)((int64_t)H * wg / nwg), R = (int)((int64_t)H * (wg + 1) / nwg) - g0;
  if (!wait()) return;
  for (int t = threadIdx.x; t < nb * R; t += NT) {
    const int b = t / R, g = g0 + (t - b * R);
    float y[MAX_TOPK];
#pragma unroll
    for (int j = 0; j < MAX_TOPK; ++j) y[j] = j < K ? bf2f(ld_ag_u16(p.ys + (size_t)s.bpair[b][j] * H + g)) : 0.0f;
    const float xr = bf2f(ld_ag_u16(p.x16 + (size_t)b * H + g));
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < MAX_TOPK; ++j)
      if (j < K) acc = bfr(acc + y[j]);
    st_ag_u16(p.x16 + (size_t)b * H + g, f2bf(xr + acc));
  }
}

// dense MLP (ref_numpy.py:149-152): gate/up + SiLU*up per sequence into h16, then down + residual
template <class WR, int B, class S, class Wait>
__device__ __forceinline__ void phase_gateup_b(const Params& p, int layer, S& s, Wait wait) {
  constexpr int KK = WR::K;
  const LayerW Lw = layer_w(p, layer);
  const int I = p.I, IS = p.Ip, nb = p.B;                 // h rows are Ip long; entries [I, Ip) stay zero
  const uint8_t* W = Lw.wgu;
  gemv_run_b<WR, 2, B>(
      I, [&](int g, int i) -> const uint8_t* { return mrow<WR>(W, (size_t)2 * g + i); }, [&](int) { return nb; },
      [&](int, int b) { return (const uint16_t*)(s.n.xs + b * KK); },
      [&](int g, int nv, const float(&v)[2][B]) {
        const int lane = lane_id();
        const float gv = lane_pick<1, B>((const float(&)[1][B])v[0]), uv = lane_pick<1, B>((const float(&)[1][B])v[1]);
        st_ag_u16(lane < nv ? p.h16d + (size_t)lane * IS + perm_stored(g, IS) : (uint16_t*)sink_of(p),
                  f2bf(bfr(bfr(silu(bfr(gv))) * bfr(uv))));
      },
      [&]() {
        if (!wait()) return false;
        build_norm_xb<KK, B>(p, false, Lw.ln2, s);
        return true;
      },
      p.nwg, p.trace, s.phase);
}

template <class WR, int B, class S, class Wait>
__device__ __forceinline__ void phase_down_b(const Params& p, int layer, S& s, Wait wait) {
  constexpr int KK = WR::K;
  static_assert(B * KK <= S::XCAP, "intermediate rows exceed the LDS budget");
  const LayerW Lw = layer_w(p, layer);
  const int H = p.H, nb = p.B, nw = p.nwg * NWAVE;
  const uint8_t* W = Lw.wd;
  gemv_run_b<WR, 1, B>(
      H, [&](int g, int) -> const uint8_t* { return mrow<WR>(W, g); }, [&](int) { return nb; },
      [&](int, int b) { return (const uint16_t*)(s.v.xs + b * KK); },
      [&](int g, int nv, const float(&v)[1][B]) {
        const int r = res_slot(g, nw);
        lane_store_b<1, B>(v, nv, [&](int, int b, float val, bool ok) {
          st_ag_u16(ok ? p.x16 + (size_t)b * H + g : (uint16_t*)sink_of(p), f2bf(s.v.xres[b][r] + bfr(val)));
        });
      },
      [&]() {
        load_res_rows<B>(p, H, false, s);
        if (!wait()) return false;
        copy_rows_lds(p.h16d, nb * KK, s.v.xs);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        return true;
      },
      p.nwg, p.trace, s.phase);
}

// P7: final norm + lm_head + greedy argmax per sequence (ref_numpy.py:155-158; vl_tiles.hip:45-89)
template <int KK, int B, class S, class Wait>
__device__ __forceinline__ void phase_head_b(const Params& p, S& s, Wait wait) {
  using WR = Bf16Row<KK>;                                 // lm_head stays bf16 in every weight type
  const int V = p.V, nb = p.B;
  const uint8_t* W = (const uint8_t*)p.lm_head;
  uint64_t best = 0;                                      // lane b: the best key of sequence b
  const bool ran = gemv_run_b<WR, 2, B>(
      (V + 1) / 2,
      [&](int g, int i) -> const uint8_t* { const int r = 2 * g + i; return r < V ? mrow<WR>(W, r) : nullptr; },
      [&](int) { return nb; }, [&](int, int b) { return (const uint16_t*)(s.n.xs + b * KK); },
      [&](int g, int nv, const float(&v)[2][B]) {
        const int lane = lane_id();
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int r = 2 * g + i;
          const float val = lane_pick<1, B>((const float(&)[1][B])v[i]);
          if (r < V && lane < nv) {
            const uint64_t key = argmax_key(bfr(val), r);
            best = key > best ? key : best;
          }
        }
      },
      [&]() {
        if (!wait()) return false;
        build_norm_xb<KK, B>(p, false, p.final_norm, s);
        if (blockIdx.x == 0 && p.dump_x)
          for (int i = threadIdx.x; i < nb * KK; i += NT)
            st_f(p.dump_x + (size_t)(p.l1 - 1) * nb * KK + i, bf2f(s.n.xr[i]));
        return true;
      },
      p.nwg, p.trace, s.phase);
  if (ran && lane_id() < nb && best)
    __hip_atomic_fetch_max(p.amax + 32 * lane_id(), best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// P7 on the matrix cores (p.mfma): 16-row tiles of the lm_head (bf16) against every sequence's final normed row,
// each tile's 4 blocks chained as the expert gate/up tiles; lane l keeps the best key of its sequence l % 16 over
// its rows, the four quads of a column are folded, and one atomic per (wave, sequence) publishes it
template <int KK, int B, class S, class Wait>
__device__ __forceinline__ void phase_head_mfma(const Params& p, S& s, Wait wait) {
  using WR = Bf16Row<KK>;                                 // lm_head stays bf16 in every weight type
  const int nb = p.B;
  const uint8_t* W = (const uint8_t*)p.lm_head;
  uint64_t best = 0;
  const bool ran = mfma_tiles<WR>(
      p, p.V / 16, [&](int t) { return mrow<WR>(W, (size_t)16 * t + (lane_id() & 15)); },
      [&](int, bool& has) -> const uint16_t* {
        const int r = lane_id() & 15;
        has = r < nb;
        return s.n.xs + (size_t)(has ? r : 0) * KK;
      },
      [&](int t, const float(&v)[4]) {
        const int r = lane_id() & 15, q = lane_id() >> 4;
        if (r < nb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint64_t key = argmax_key(bfr(v[i]), 16 * t + 4 * q + i);
            best = key > best ? key : best;
          }
      },
      [&]() {
        if (!wait()) return false;
        build_norm_xb<KK, B>(p, false, p.final_norm, s);
        if (blockIdx.x == 0 && p.dump_x)
          for (int i = threadIdx.x; i < nb * KK; i += NT)
            st_f(p.dump_x + (size_t)(p.l1 - 1) * nb * KK + i, bf2f(s.n.xr[i]));
        return true;
      },
      s.phase);
  if (!ran) return;
#pragma unroll
  for (int m = 16; m < 64; m <<= 1) {                     // fold the quads: lanes r, r + 16, r + 32, r + 48
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)best, m, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(best >> 32), m, 64);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    best = o > best ? o : best;
  }
  if (lane_id() < nb && best)
    __hip_atomic_fetch_max(p.amax + 32 * lane_id(), best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <class Wait>
__device__ __forceinline__ void phase_token_b(const Params& p, Wait wait) {
  if (!wait()) return;
  const int b = threadIdx.x;
  if (blockIdx.x == 0 && b < p.B) {
    const uint64_t key = ld_ag64(p.amax + 32 * b);
    int32_t tok = (int32_t)(0xFFFFFFFFu - (uint32_t)key);
    if (key == 0 || tok < 0 || tok >= p.V) {              // no finite logit was seen: flag it, keep the id valid
      st_ag_i(p.abort_word, 3);
      tok = 0;
    }
    const size_t row = (size_t)b * p.tok_stride;
    st_ag_i(p.out_tokens + row + p.posb[b], tok);
    if ((p.write_next >> b) & 1) st_ag_i(p.tokens + row + p.posb[b] + 1, tok);
  }
}

// ---------------------------------------------------------------- batched persistent kernel
template <int H, int KA, int KM, bool MOE, int EC, bool FP8, int B>
__device__ __forceinline__ void fused_body_b(const Params& p) {
  __shared__ SmemB<B> s;
  if (threadIdx.x == 0) s.abort = 0;
  __syncthreads();
  int k = 0;
  auto wait = [&]() { return grid_wait(p, k, s); };
  if (p.trace && threadIdx.x == 0) *(MK_G uint64_t*)(p.trace + (size_t)blockIdx.x * 3) = __builtin_amdgcn_s_memrealtime();
  s.phase = 0;
  // the matrix-core forms (p.mfma, set by the host for MoE handles of batch capacity >= 8 whose shapes take whole
  // tiles): the dense projections, the router, the expert rows and the lm_head in 16-row tiles against up to 16
  // sequence columns
  constexpr int TB = FP8 ? 1024 : 512;
  constexpr bool TILES = MOE && B >= 8 && H % TB == 0 && KA % TB == 0 && H / TB <= NWAVE && KA / TB <= NWAVE &&
                        H / 512 <= NWAVE && EC % 16 == 0 && KM % 256 == 0 && KM <= 4096;
  for (int layer = p.l0; layer < p.l1; ++layer) {
    if constexpr (TILES) {
      if (p.mfma) phase_qkv_mfma<RowOf<FP8, H>, B>(p, layer, s, wait);
      else phase_qkv_b<RowOf<FP8, H>, B>(p, layer, s, wait);
    } else {
      phase_qkv_b<RowOf<FP8, H>, B>(p, layer, s, wait);
    }
    if (s.abort) return;
    grid_arrive(p, k, s);
    phase_attn_b<B>(p, layer, s, wait);
    if (s.abort) return;
    grid_arrive(p, k, s);
    phase_attn_merge_b<B>(p, s, wait);
    if (s.abort) return;
    grid_arrive(p, k, s);
    if constexpr (TILES) {
      if (p.mfma) phase_oproj_mfma<RowOf<FP8, KA>, B>(p, layer, s, wait);
      else phase_oproj_b<RowOf<FP8, KA>, B>(p, layer, s, wait);
    } else {
      phase_oproj_b<RowOf<FP8, KA>, B>(p, layer, s, wait);
    }
    if (s.abort) return;
    grid_arrive(p, k, s);
    if constexpr (MOE) {
      if constexpr (TILES) {
        if (p.mfma) phase_router_mfma<H, B, EC>(p, layer, s, wait);
        else phase_router_b<H, B>(p, layer, s, wait);
      } else {
        phase_router_b<H, B>(p, layer, s, wait);
      }
      if (s.abort) return;
      grid_arrive(p, k, s);
      if constexpr (TILES) {
        if (p.mfma) phase_expert_up_mfma<RowOf<FP8, H>, B, EC>(p, layer, s, wait);
        else phase_expert_up_b<RowOf<FP8, H>, B, EC>(p, layer, s, wait);
      } else {
        phase_expert_up_b<RowOf<FP8, H>, B, EC>(p, layer, s, wait);
      }
      if (s.abort) return;
      grid_arrive(p, k, s);
      if constexpr (TILES) {
        if (p.mfma) {
          phase_expert_down_mfma<RowOf<FP8, KM>, B>(p, layer, s, wait);
          if (s.abort) return;
          grid_arrive(p, k, s);
          phase_combine_mfma<B>(p, s, wait);
        } else {
          phase_expert_down_b<RowOf<FP8, KM>, B>(p, layer, s, wait);
        }
      } else {
        phase_expert_down_b<RowOf<FP8, KM>, B>(p, layer, s, wait);
      }
      if (s.abort) return;
      grid_arrive(p, k, s);
    } else {
      phase_gateup_b<RowOf<FP8, H>, B>(p, layer, s, wait);
      if (s.abort) return;
      grid_arrive(p, k, s);
      phase_down_b<RowOf<FP8, KM>, B>(p, layer, s, wait);
      if (s.abort) return;
      grid_arrive(p, k, s);
    }
  }
  if (p.do_head) {
    if constexpr (TILES) {
      if (p.mfma) phase_head_mfma<H, B>(p, s, wait);
      else phase_head_b<H, B>(p, s, wait);
    } else {
      phase_head_b<H, B>(p, s, wait);
    }
    if (s.abort) return;
    grid_arrive(p, k, s);
    phase_token_b(p, wait);
  }
}

// batched shapes: name, H, KA, KM, MoE, E, fp8 weights, batch capacity (the host picks the smallest capacity that
// holds its batch); one translation unit per list (mk_batch_bf16.hip, mk_batch_fp8.hip)
#define MK_BATCH_SHAPES_BF16(X)                                                      \
  X(etxmk_fused_b4_h2048_a4096_moe768_e128, 2048, 4096, 768, true, 128, false, 4)   \
  X(etxmk_fused_b16_h2048_a4096_moe768_e128, 2048, 4096, 768, true, 128, false, 16) \
  X(etxmk_fused_b4_h512_a512_moe256_e16, 512, 512, 256, true, 16, false, 4)         \
  X(etxmk_fused_b16_h512_a512_moe256_e16, 512, 512, 256, true, 16, false, 16)       \
  X(etxmk_fused_b4_h512_a512_mlp1024, 512, 512, 1024, false, 0, false, 4)           \
  X(etxmk_fused_b4_h4096_a4096_mlp12288, 4096, 4096, 12288, false, 0, false, 4)
#define MK_BATCH_SHAPES_FP8(X)                                                          \
  X(etxmk_fused_fp8_b4_h2048_a4096_moe768_e128, 2048, 4096, 768, true, 128, true, 4)   \
  X(etxmk_fused_fp8_b16_h2048_a4096_moe768_e128, 2048, 4096, 768, true, 128, true, 16) \
  X(etxmk_fused_fp8_b4_h512_a512_moe256_e16, 512, 512, 256, true, 16, true, 4)         \
  X(etxmk_fused_fp8_b16_h512_a512_moe256_e16, 512, 512, 256, true, 16, true, 16)       \
  X(etxmk_fused_fp8_b4_h512_a512_mlp1024, 512, 512, 1024, false, 0, true, 4)
#define MK_BATCH_KERNEL(name, H, KA, KM, MOE, EC, FP8, B) \
  extern "C" __global__ void __launch_bounds__(NT, 1) name(Params p) { fused_body_b<H, KA, KM, MOE, EC, FP8, B>(p); }
#define MK_BATCH_DECL(name, H, KA, KM, MOE, EC, FP8, B) \
  extern "C" __global__ void __launch_bounds__(NT, 1) name(Params p);

}  // namespace mk
