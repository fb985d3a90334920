#pragma once
// Batch-small decode step for gfx950 (MI355X): one persistent cooperative launch per token that runs every
// layer's phases back to back, separated by split grid barriers (arrive at the end of a phase, wait inside the
// next one after its weight loads are in flight), or (unfused mode) one ordinary launch per phase with the same
// device functions.
//
// Reference path (relative to the reference checkout): examples/llm/ref_numpy.py:105-158 is the numerical
// specification; examples/llm/tiles.hip:23-357 and etx/codegen/kernel.py:471-605 are the tile bodies and
// the persistent worker loop this file replaces.
//
// Phases of one layer (MoE):   P1 norm + QKV GEMV | P2 q/k norm, RoPE, paged KV append, chunked attention with
//                              a last-arriver merge | P3 O projection + residual | P4 norm + router GEMV |
//                              P5 top-k + expert gate/up GEMV + SiLU*up | P6 expert down GEMV, weight, combine, residual
// Dense layers replace P4-P6 by gate/up (+SiLU*up) and down (+residual).  Head: final norm + lm_head GEMV with
// a 64-bit packed argmax key, then the token write.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include <type_traits>

#include "etxmk.h"
#include "mk_numerics.h"

namespace mk {

constexpr int NT = 512;                 // threads per workgroup: 8 waves, two per SIMD
constexpr int NWAVE = NT / 64;
constexpr int CHUNK = 64;               // attention positions per chunk (one lane per position)
constexpr int HDIM = 128;               // head dim handled by the attention phase
constexpr int MAX_H = 4096;
constexpr int MAX_K = 12288;
constexpr int MAX_CTX = 8192;
constexpr int MAX_CHUNKS = MAX_CTX / CHUNK;  // at most two per lane in the attention merge
static_assert(MAX_CHUNKS <= 128, "the attention merge holds two chunks per lane");
constexpr int MAX_G = 16;               // q heads per kv head
constexpr int MAX_E = 256;
constexpr int MAX_TOPK = 8;
constexpr int PART = HDIM + 2;          // attention partial: a[HD], m, l
constexpr int QKVW_BYTES = 81920;       // the workgroup's rows of the next layer's QKV matrix, staged in LDS
constexpr int MAX_B = 16;               // sequences per batched step
constexpr int SINK_WAVES = 2048;        // waves with a private store sink (more share them modulo)

// one layer's tensors; matrices are byte addresses of rows in their format (Bf16Row / Fp8Row below)
struct LayerW {
  const uint16_t *ln1, *ln2, *qn, *kn;            // DeepSeek-V2: kn is the kv_a_layernorm weight [kv_lora]
  const uint8_t *wqkv, *wo, *wr, *w13, *w2, *wgu, *wd;
  uint16_t *kc, *vc;                              // DeepSeek-V2: kc is the latent cache, vc unused
  const uint8_t *wuk, *wuv, *wsgu, *wsd;          // DeepSeek-V2: W_UK^T [NH][kv_lora][qk_nope], W_UV [NH*v_head][kv_lora],
                                                  // shared experts gate/up [2*SI][H] (interleaved) and down [H][SI]
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
  float* apart;                         // [NH][MAX_CHUNKS][PART] attention partials
  uint32_t* acnt;                       // [NKV] chunk arrival counters, 256 B apart (zero between steps)
  uint64_t* amax;
  uint32_t* bar;
  int32_t* abort_word;
  const int32_t* host_stop;             // the host's stop request (pinned host memory; etxmk_abort / a sync timeout)
  int32_t* tokens;
  int32_t* out_tokens;
  float* dump_x;
  int32_t* dump_ids;
  float* dump_wts;
  float* dump_logits;
  uint64_t* trace;                      // optional: [phase][workgroup][wait done, arrive, loads issued] stamps
  int pos, write_next, l0, l1, do_embed, do_head;
  int qkv_rows;                         // > 0: QKV rows per workgroup, the first qkv_lds_rows of them staged in LDS
  int qkv_lds_rows;                     // one layer ahead, the rest loaded before the QKV phase's wait (fused mode)
  uint32_t bar_base;
  int nwg;
  uint64_t spin_ticks;
  uint32_t poll_mask;                   // a waiting workgroup checks the abort and stop words when (polls & mask) == 0
  // batched steps: per-sequence activations are [B][...] rows of the buffers above; tokens / out_tokens rows are
  // tok_stride long; btab rows nbps long; amax entries 256 bytes apart
  int B, nbps, tok_stride;
  int pf;                               // prefill: rows b are positions posb[0] + b of one sequence (btab and
                                        // tokens point at its rows, nbps = tok_stride = 0)
  int mfma;                             // batched projections and experts on the matrix cores (handles of batch
                                        // capacity >= 8 whose shapes take whole tiles)
  uint16_t* ys;                         // matrix-core expert down: [pairs][H] weighted outputs, bf16, for the combine
  uint16_t* x16;                        // [B][H] residual, bf16
  uint16_t* o16;                        // [B][NH*HD] attention output, bf16 lane-permuted
  uint16_t* h16;                        // MoE [pairs][MI] / dense [B][I] MLP activations, bf16 lane-permuted
  int posb[MAX_B];                      // sequence b's position
  int ibase[MAX_B + 1];                 // attention items of the sequences before b (NKV * chunks each)
  int nqkv;                             // rows of the fused QKV matrix (DeepSeek-V2: q_proj and kv_a_proj_with_mqa)
  uint16_t* h16d;                       // dense MLP activations [B][Ip] (Ip: I rounded up to the row format; pads zero)
  int Ip;
  // DeepSeek-V2 (arch 1)
  int arch, first_dense, SI;            // SI = n_shared * MI, the shared experts' width
  float routed_scale;
  float* qc;                            // [L][B][NH][kv_lora] absorbed queries, fp32
  uint16_t* h16s;                       // [B][SI] shared experts' activations, bf16 lane-permuted
  float* sink;                          // [SINK_WAVES][64]: where a batched GEMV's lanes with no value store (one
                                        // word per wave, 256 bytes apart), so
                                        // every epilogue is one store per lane and the load waits stay exact
};

// the attention phase's LDS (one (sequence, kv head, chunk) item at a time)
// CPI chunks of 64 positions per attention item (one tile pair each)
template <int CPI>
struct AttnTilesT {
  static constexpr int cpi = CPI;
  u32x4 kt[CPI][HDIM / 8][CHUNK];       // K tiles: [chunk][8-dim group][position in chunk], 16 bytes each
  u32x4 vt[CPI][CHUNK / 8][2][CHUNK];   // V tiles: [chunk][8-position group][dim half][dim in half], 16 bytes each
  float p[MAX_G][2 * MAX_CHUNKS];       // merge: chunk weights, then chunk sums, per head
};
using AttnTiles = AttnTilesT<1>;

struct Smem {
  union {
    struct {
      float xf[MAX_H];                  // residual (natural order, fp32)
      alignas(16) uint16_t xs[MAX_K];   // GEMV input vector(s), lane-permuted bf16
    } g;
    AttnTiles a;
  };
  alignas(16) u32x4 qkvw[QKVW_BYTES / 16];  // next layer's QKV rows [row of this workgroup][K/8], lane-permuted
  float rs;
  int32_t ids[NWAVE][MAX_TOPK];         // routing, one private copy per wave (no workgroup barrier needed)
  float wts[NWAVE][MAX_TOPK];
  int32_t order[NWAVE][MAX_TOPK];
  float lg[MAX_E];                      // the router logits, read once per workgroup
  int32_t abort;
  int32_t last;
  int32_t phase;                        // arrivals so far (the current phase index), for trace stamps
};

// The lane.  Translation units that define MK_LANE_OPAQUE (the batched kernels) put it behind an empty volatile asm
// so that what is computed from it stays where it is computed: the compiler cannot hoist the asm, so no
// lane-dependent offset or address is lifted out of the layer loop to hold registers through every phase.  With
// plain threadIdx.x & 63 such hoisted values pushed the batch-16 kernels to 256 VGPRs with 31 to 78 spilled, and a
// spill reloaded inside a pipelined loop waits for every load still in flight (vmcnt counts in order): +8 us per layer
// in the batch-16 attention phase.  The single-sequence kernels fit without it and run 2% faster with the hoisting.
__device__ __forceinline__ int lane_id() {
  int l = threadIdx.x & 63;
#ifdef MK_LANE_OPAQUE
  asm volatile("" : "+v"(l));
#endif
  return l;
}
// one layer's pointer table, read through the constant address space (scalar loads)
__device__ __forceinline__ LayerW layer_w(const Params& p, int layer) {
  static_assert(sizeof(LayerW) % 8 == 0, "pointer table");
  const __attribute__((address_space(4))) uint64_t* src = (const __attribute__((address_space(4))) uint64_t*)(p.layers + layer);
  LayerW r;
  uint64_t* dst = (uint64_t*)&r;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(LayerW) / 8); ++i) dst[i] = src[i];
  return r;
}
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }
// the wave index as a value the compiler knows is uniform (kept in a scalar register)
__device__ __forceinline__ int wave_u() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// ---------------------------------------------------------------- grid barrier (split: arrive / wait)
// Monotonic counters (never reset): the j-th arrival of this launch publishes generation bar_base + j + 1.
// Arrival is hierarchical to spread the atomics over 8 lines: workgroup w counts into group w % 8; the last
// arrival of a group counts into the global word; the last group's last arrival writes the generation into
// the 8 release flags, and every workgroup polls its group's flag.
// Visibility: every value another workgroup reads is written with an agent-scope (sc1) store and read with an
// agent-scope load; each wave waits for its own stores to complete (s_waitcnt 0) before the workgroup barrier
// that precedes the arrival, so no L2 write-back or invalidate is needed.  The wait is bounded by a wall-clock
// limit; on expiry the abort word is set and every workgroup leaves.  Every 256 polls (poll_mask + 1) a waiting
// workgroup also checks the clock, the abort word and the host's stop word: either makes it leave, and a stop request is copied into the abort word so
// the rest of the grid leaves at its next check.
template <class S>
__device__ __forceinline__ void grid_arrive(const Params& p, int& k, S& s) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    s.phase = k + 1;
    if (p.trace) *(MK_G uint64_t*)(p.trace + ((size_t)k * p.nwg + blockIdx.x) * 3 + 1) = __builtin_amdgcn_s_memrealtime();
    const int g = blockIdx.x & 7;
    const uint32_t ng = (uint32_t)(p.nwg - g + 7) / 8u;
    const uint32_t gen = p.bar_base + (uint32_t)k + 1u;
    const uint32_t old = __hip_atomic_fetch_add(p.bar + 64 * g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old + 1u == gen * ng) {
      const uint32_t o2 = __hip_atomic_fetch_add(p.bar + 64 * 8, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (o2 + 1u == gen * 8u)
        for (int j = 0; j < 8; ++j) __hip_atomic_store(p.bar + 64 * (9 + j), gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  ++k;
}

// wait until the k-th arrival's generation is published (nothing to wait for when k == 0)
template <class S>
__device__ __forceinline__ bool grid_wait(const Params& p, int k, S& s) {
  if (k == 0) return true;
  if (threadIdx.x == 0) {
    const uint32_t gen = p.bar_base + (uint32_t)k;
    const uint32_t* flag = p.bar + 64 * (9 + (blockIdx.x & 7));
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    int ab = 0;
    uint32_t polls = 0;
    while ((int32_t)(__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - gen) < 0) {
      __builtin_amdgcn_s_sleep(1);
      if ((++polls & p.poll_mask) == 0) {
        if (ld_ag_i(p.abort_word) != 0) { ab = 1; break; }
        if (p.host_stop && ld_sys_i(p.host_stop) != 0) {   // the host asked the step to stop: tell the grid
          st_ag_i(p.abort_word, 1);
          ab = 1;
          break;
        }
        if (__builtin_amdgcn_s_memrealtime() - t0 > p.spin_ticks) {
          st_ag_i(p.abort_word, 2);
          ab = 1;
          break;
        }
      }
    }
    s.abort = ab;
    if (p.trace) *(MK_G uint64_t*)(p.trace + ((size_t)k * p.nwg + blockIdx.x) * 3) = __builtin_amdgcn_s_memrealtime();
  }
  __syncthreads();
  return s.abort == 0;
}

// ---------------------------------------------------------------- vectors into LDS
// Each helper issues all of a thread's global loads before it uses any of them (one memory latency, not one
// per element).

// x (n fp32, agent-scope) -> dst[n] natural order
__device__ __forceinline__ void load_x(const float* xg, int n, float* dst) {
  constexpr int PER = (MAX_H / 2 + NT - 1) / NT;
  const int n2 = n / 2;
  uint64_t v[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = threadIdx.x + j * NT;
    if (i < n2) v[j] = ld_ag64((const uint64_t*)xg + i);
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = threadIdx.x + j * NT;
    if (i < n2) { dst[2 * i] = bits2f((uint32_t)v[j]); dst[2 * i + 1] = bits2f((uint32_t)(v[j] >> 32)); }
  }
}
// a bf16 row of n elements (the embedding row) -> dst[n] fp32
__device__ __forceinline__ void load_row_bf16(const uint16_t* row, int n, float* dst) {
  constexpr int PER = (MAX_H / 8 + NT - 1) / NT;
  const int n8 = n / 8;
  u32x4 v[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = threadIdx.x + j * NT;
    if (i < n8) v[j] = ld16(row + 8 * i);
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = threadIdx.x + j * NT;
    if (i < n8)
#pragma unroll
      for (int e = 0; e < 4; ++e) { dst[8 * i + 2 * e] = bf_lo(v[j][e]); dst[8 * i + 2 * e + 1] = bf_hi(v[j][e]); }
  }
}
// the residual entering a phase: the embedding row of the step's token for the first layer, else x
__device__ __forceinline__ void load_residual(const Params& p, bool first, int tok, float* dst) {
  if (first) load_row_bf16(p.embed + (size_t)tok * p.H, p.H, dst);
  else load_x(p.x, p.H, dst);
}

// x -> s.g.xf; RMSNorm with weight w, lane-permuted bf16 -> s.g.xs (ref_numpy.py:71-73:
// r = 1/sqrt(mean(x^2) + eps), out = bfr(w * bfr(x * r)); the sum of squares in dot order).
// Thread t writes stored chunk t (8 stored positions = 16 bytes of LDS).
template <int H>
__device__ __forceinline__ void build_norm_x(const Params& p, const float* xg, const uint16_t* xrow, const uint16_t* w,
                                             Smem& s) {
  constexpr int N8 = H / 8, PER = (N8 + NT - 1) / NT;
  uint16_t wv[PER][8];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = threadIdx.x + j * NT;
    if (c < N8)
#pragma unroll
      for (int e = 0; e < 8; ++e) wv[j][e] = ld_u16(w + perm_logical(8 * c + e, H));
  }
  if (xrow) load_row_bf16(xrow, H, s.g.xf);
  else load_x(xg, H, s.g.xf);
  __syncthreads();
  if (wave_id() == 0) {
    float acc = 0.0f;
#pragma unroll 8
    for (int k = lane_id(); k < H; k += 64) acc = __builtin_fmaf(s.g.xf[k], s.g.xf[k], acc);
    acc = wave_sum(acc);
    if (lane_id() == 0) s.rs = 1.0f / __builtin_sqrtf(acc / (float)H + p.eps);
  }
  __syncthreads();
  const float r = s.rs;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = threadIdx.x + j * NT;
    if (c < N8) {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const int k0 = perm_logical(8 * c + e, H), k1 = perm_logical(8 * c + e + 1, H);
        const uint32_t b0 = f2bf(bfr(bf2f(wv[j][e]) * bfr(s.g.xf[k0] * r)));
        const uint32_t b1 = f2bf(bfr(bf2f(wv[j][e + 1]) * bfr(s.g.xf[k1] * r)));
        o[e / 2] = b0 | (b1 << 16);
      }
      *(u32x4*)(s.g.xs + 8 * c) = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
  __syncthreads();
}

// nv bf16-valued fp32 vectors of length K (agent-scope, contiguous) -> lane-permuted bf16 at dst (contiguous)
template <int K, int MAXV>
__device__ __forceinline__ void load_vec_perm(const float* src, int nv, uint16_t* dst) {
  constexpr int C8 = K / 8, PER = (MAXV * C8 + NT - 1) / NT;
  float v[PER][8];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = threadIdx.x + j * NT;
    if (c < nv * C8) {
      const int vec = c / C8, q = 8 * (c - vec * C8);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = ld_ag(src + (size_t)vec * K + perm_logical(q + e, K));
    }
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = threadIdx.x + j * NT;
    if (c < nv * C8) {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) o[e / 2] = (uint32_t)f2bf(v[j][e]) | ((uint32_t)f2bf(v[j][e + 1]) << 16);
      *(u32x4*)(dst + 8 * c) = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
}

// ---------------------------------------------------------------- streaming GEMV
template <int K>
struct KS {
  static_assert(K % 64 == 0, "row length must be a multiple of 64");
  static constexpr int KB = K / 512;
  static constexpr int TM = (K % 512) / 64;      // stored elements per lane in the tail block
  static_assert(TM % 2 == 0, "tail block must give each lane whole dwords");
  static constexpr int TW = TM / 2;
  static constexpr int REGS = 4 * KB + TW;       // VGPRs one row occupies in flight
};

template <int K>
struct RowRegs {
  u32x4 w[KS<K>::KB > 0 ? KS<K>::KB : 1];
  uint32_t t[KS<K>::TW > 0 ? KS<K>::TW : 1];
};

template <int K>
__device__ __forceinline__ void load_row(RowRegs<K>& r, const uint16_t* row, int lane) {
#pragma unroll
  for (int b = 0; b < KS<K>::KB; ++b) r.w[b] = ld_nt16(row + 512 * b + lane * 8);
#pragma unroll
  for (int t = 0; t < KS<K>::TW; ++t)
    r.t[t] = ld_nt4(row + 512 * KS<K>::KB + lane * KS<K>::TM + 2 * t);
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
  return wave_sum(acc);
}

// Long rows (more than 16 blocks of 512): streamed in segments of SEG blocks (a divisor of the block count near
// 8), the next segment's loads in flight while the current one is accumulated; the accumulation order is the same
// as dot_row's.
constexpr int seg_of(int kb) {
  for (int s = 8; s >= 4; --s)
    if (kb % s == 0) return s;
  for (int s = 9; s <= 12; ++s)
    if (kb % s == 0) return s;
  return 0;
}
template <int K>
__device__ __forceinline__ float dot_row_long(const uint16_t* row, const uint16_t* xs, int lane) {
  constexpr int SEG = seg_of(KS<K>::KB), NS = SEG ? KS<K>::KB / SEG : 0;
  static_assert(SEG > 0 && KS<K>::TW == 0, "long rows are whole segments of 4 to 12 blocks");
  u32x4 A[SEG], B[SEG];
  float acc = 0.0f;
  auto ld = [&](u32x4(&R)[SEG], int sg) {
#pragma unroll
    for (int b = 0; b < SEG; ++b) R[b] = ld_nt16(row + 512 * (sg * SEG + b) + lane * 8);
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
  return wave_sum(acc);
}

// fp8 rows (etxmk_config.wdtype = ETXMK_W_FP8): K e4m3 codes stored lane-permuted in blocks of 1024 (lane l's 16
// bytes of a block are the logical elements l, l+64, ..., l+960; a last block of 64m elements gives each lane m),
// then the row's fp32 scale, rows K + 16 bytes apart.  The input vector keeps its bf16 layout (blocks of 512), so
// a block's first 8 codes pair with the lane's 8 elements of one 512-block and the next 8 with the following one.
template <int K>
struct KS8 {
  static_assert(K % 256 == 0, "fp8 rows are whole 256-element quarters of a block");
  static constexpr int KB = K / 1024;
  static constexpr int T = K % 1024;             // tail block length
  static constexpr int TM = T / 64;              // codes per lane in the tail (4, 8 or 12)
  static constexpr int TW = TM / 4;
  static constexpr int REGS = 4 * KB + TW + 1;   // VGPRs one row occupies in flight (with its scale)
};

template <int K>
struct RowRegs8 {
  u32x4 w[KS8<K>::KB > 0 ? KS8<K>::KB : 1];
  uint32_t t[KS8<K>::TW > 0 ? KS8<K>::TW : 1];
  float sc;
};

template <int K>
__device__ __forceinline__ void load_row8(RowRegs8<K>& r, const uint8_t* row, int lane) {
#pragma unroll
  for (int b = 0; b < KS8<K>::KB; ++b) r.w[b] = ld_nt16(row + 1024 * b + lane * 16);
#pragma unroll
  for (int t = 0; t < KS8<K>::TW; ++t) r.t[t] = ld_nt4(row + 1024 * KS8<K>::KB + lane * KS8<K>::TM + 4 * t);
  r.sc = ld_f((const float*)(row + K));
}

// the 16 input elements that pair with lane `lane`'s codes of fp8 block j (or its tail), as fp32
template <int K>
__device__ __forceinline__ void x_of_fp8_block(const uint16_t* xs, int j, int lane, float (&xv)[16]) {
  if (j < KS8<K>::KB || KS8<K>::T >= 512) {
    const u32x4 a = *(const u32x4*)(xs + 1024 * j + lane * 8);
#pragma unroll
    for (int e = 0; e < 4; ++e) { xv[2 * e] = bf_lo(a[e]); xv[2 * e + 1] = bf_hi(a[e]); }
  }
  if (j < KS8<K>::KB) {
    const u32x4 b = *(const u32x4*)(xs + 1024 * j + 512 + lane * 8);
#pragma unroll
    for (int e = 0; e < 4; ++e) { xv[8 + 2 * e] = bf_lo(b[e]); xv[9 + 2 * e] = bf_hi(b[e]); }
  } else if constexpr (KS8<K>::T == 768) {                // 512 + a 256 bf16 tail (4 per lane)
    const uint64_t b = *(const uint64_t*)(xs + 1024 * j + 512 + lane * 4);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t w = (uint32_t)(b >> (32 * e));
      xv[8 + 2 * e] = bf_lo(w);
      xv[9 + 2 * e] = bf_hi(w);
    }
  } else if constexpr (KS8<K>::T == 256) {                // a 256 bf16 tail (4 per lane)
    const uint64_t b = *(const uint64_t*)(xs + 1024 * j + lane * 4);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t w = (uint32_t)(b >> (32 * e));
      xv[2 * e] = bf_lo(w);
      xv[2 * e + 1] = bf_hi(w);
    }
  }
}
// the codes of block j (or the tail) decoded to fp32 (hardware OCP e4m3 conversion, exact)
template <int K>
__device__ __forceinline__ void w_of_fp8_block(const RowRegs8<K>& r, int j, float (&wv)[16]) {
  constexpr int NW = KS8<K>::TW;
  auto dec4 = [&](uint32_t d, int e0) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, true);
    wv[e0] = lo[0]; wv[e0 + 1] = lo[1]; wv[e0 + 2] = hi[0]; wv[e0 + 3] = hi[1];
  };
  if (j < KS8<K>::KB) {
#pragma unroll
    for (int d = 0; d < 4; ++d) dec4(r.w[j][d], 4 * d);
  } else {
#pragma unroll
    for (int d = 0; d < NW; ++d) dec4(r.t[d], 4 * d);
  }
}

// fp8 row dot: lane order as dot_row (blocks ascending, a lane's elements ascending), then wave_sum, then the scale
template <int K>
__device__ __forceinline__ float dot_row8(const RowRegs8<K>& r, const uint16_t* xs, int lane) {
  constexpr int NB = KS8<K>::KB + (KS8<K>::T > 0 ? 1 : 0);
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int n = j < KS8<K>::KB ? 16 : KS8<K>::TM;
    float wv[16], xv[16];
    w_of_fp8_block<K>(r, j, wv);
    x_of_fp8_block<K>(xs, j, lane, xv);
#pragma unroll
    for (int e = 0; e < 16; ++e)
      if (e < n) acc = __builtin_fmaf(wv[e], xv[e], acc);
  }
  return wave_sum(acc) * r.sc;
}

// Row formats of the streamed matrices: the register image of one row in flight, its load and its dot with the
// input vector in LDS.  The GEMV engine and the phases are written once over these.
template <int K_>
struct Bf16Row {
  static constexpr int K = K_;
  static constexpr bool FP8 = false;
  static constexpr bool LONG = KS<K>::KB > 16;   // streamed in segments (dot_row_long), not held in registers
  static constexpr size_t STRIDE = 2 * (size_t)K;
  static constexpr int REGS = KS<K>::REGS;
  using Regs = RowRegs<K>;
  __device__ static void load(Regs& r, const uint8_t* row, int lane) { load_row<K>(r, (const uint16_t*)row, lane); }
  __device__ static float dot(const Regs& r, const uint16_t* xs, int lane) { return dot_row<K>(r, xs, lane); }
  __device__ static float dot_long(const uint8_t* row, const uint16_t* xs, int lane) {
    if constexpr (LONG) return dot_row_long<K>((const uint16_t*)row, xs, lane);
    else return 0.0f;
  }
};
// An empty asm reading every register of a row buffer: the compiler's wait for the buffer's loads lands here, on
// every path.  Without it the first uses sit in conditional code, the skip path leaves the buffer pending, and
// the next issue into neighbouring registers waits for loads still streaming.
template <int K>
__device__ __forceinline__ void settle(const RowRegs<K>& r) {
#pragma unroll
  for (int b = 0; b < KS<K>::KB; ++b) asm volatile("" ::"v"(r.w[b]));
#pragma unroll
  for (int t = 0; t < KS<K>::TW; ++t) asm volatile("" ::"v"(r.t[t]));
}
template <int K>
__device__ __forceinline__ void settle(const RowRegs8<K>& r) {
#pragma unroll
  for (int b = 0; b < KS8<K>::KB; ++b) asm volatile("" ::"v"(r.w[b]));
#pragma unroll
  for (int t = 0; t < KS8<K>::TW; ++t) asm volatile("" ::"v"(r.t[t]));
  asm volatile("" ::"v"(r.sc));
}

template <int K_>
struct Fp8Row {
  static constexpr int K = K_;
  static constexpr bool FP8 = true;
  static constexpr bool LONG = false;
  static_assert(K <= 8192, "fp8 rows are held in registers");
  static constexpr size_t STRIDE = (size_t)K + 16;
  static constexpr int REGS = KS8<K>::REGS;
  using Regs = RowRegs8<K>;
  __device__ static void load(Regs& r, const uint8_t* row, int lane) { load_row8<K>(r, row, lane); }
  __device__ static float dot(const Regs& r, const uint16_t* xs, int lane) { return dot_row8<K>(r, xs, lane); }
  __device__ static float dot_long(const uint8_t*, const uint16_t*, int) { return 0.0f; }
};
template <bool FP8, int K>
using RowOf = typename std::conditional<FP8, Fp8Row<K>, Bf16Row<K>>::type;
// row r of a matrix stored in format WR
template <class WR>
__device__ __forceinline__ const uint8_t* mrow(const uint8_t* base, size_t r) { return base + r * WR::STRIDE; }

// Groups of NR rows are dealt round-robin to the grid's waves (group g to global wave g mod nw).  A wave loads up
// to D of its groups at once (about 96 VGPRs of weights), then reduces them; the first batch is issued before
// `prologue` runs, so the weight stream overlaps the grid-barrier wait and the input-vector build that the
// prologue does.  Every thread calls prologue() exactly once (it may synchronise the workgroup); it returns false
// to abandon the phase.  rowf(g, i) gives row i of group g (nullptr when absent), xf(i) its LDS input vector,
// epi(g, v) consumes the NR dot products (every lane holds them).  All group logic is wave-uniform.
template <class WR, int NR, class RowF, class XF, class EpiF, class Pro>
__device__ __forceinline__ bool gemv_run(int ngroups, RowF rowf, XF xf, EpiF epi, Pro prologue, int nwg,
                                         uint64_t* trace = nullptr, int s_phase = 0) {
  const int lane = lane_id();
  const int gw = blockIdx.x * NWAVE + wave_u(), nw = nwg * NWAVE;
  if constexpr (WR::LONG) {
    if (!prologue()) return false;
    for (int g = gw; g < ngroups; g += nw) {
      float v[NR];
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        const uint8_t* rp = rowf(g, i);
        v[i] = rp ? WR::dot_long(rp, xf(i), lane) : 0.0f;
      }
      epi(g, v);
    }
    return true;
  } else {
    constexpr int RPG = NR * WR::REGS;
    constexpr int D = (96 / RPG) < 1 ? 1 : (96 / RPG) > 8 ? 8 : (96 / RPG);
    typename WR::Regs R[D][NR];
    auto issue = [&](int g0) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int g = g0 + d * nw;
        if (g < ngroups) {
#pragma unroll
          for (int i = 0; i < NR; ++i) {
            const uint8_t* rp = rowf(g, i);
            if (rp) WR::load(R[d][i], rp, lane);
          }
        }
      }
    };
    int g0 = gw;
    issue(g0);
    if (trace && threadIdx.x == 0)
      *(MK_G uint64_t*)(trace + ((size_t)s_phase * nwg + blockIdx.x) * 3 + 2) = __builtin_amdgcn_s_memrealtime();
    if (!prologue()) return false;
    while (g0 < ngroups) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int g = g0 + d * nw;
        if (g < ngroups) {
          float v[NR];
#pragma unroll
          for (int i = 0; i < NR; ++i) {
            const uint8_t* rp = rowf(g, i);
            v[i] = rp ? WR::dot(R[d][i], xf(i), lane) : 0.0f;
          }
          epi(g, v);
        }
      }
      g0 += D * nw;
      if (g0 < ngroups) issue(g0);
    }
    return true;
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
// Every phase takes `wait`, the grid-barrier wait for its inputs (a no-op in unfused mode), and calls it exactly
// once from every thread, as late as its data dependences allow.
// the step's input token; an id outside the vocabulary (only possible from corrupted state) reads row 0
__device__ __forceinline__ int token_of(const Params& p) {
  const int t = ld_ag_i(p.tokens + p.pos);
  return (t >= 0 && t < p.V) ? t : 0;
}

// The QKV rows of layer `layer` that this workgroup computes are [b*R, b*R + R), R = p.qkv_rows; the first
// S = p.qkv_lds_rows of them go HBM -> LDS as stored (lane-permuted), issued from the O projection of the layer
// before: that stream overlaps the attention, router and MLP phases, whose memory traffic leaves room, and the QKV
// phase then reads them from LDS.  Wave w copies rows w, w + 8, ...; each wave reads back only the rows it copied,
// after its own wait.
template <int KK>
__device__ __forceinline__ void qkv_to_lds(const Params& p, int layer, Smem& s) {
  static_assert(KK % 512 == 0, "LDS-staged QKV rows are whole 512-element blocks");
  const LayerW Lw = layer_w(p, layer);
  const int rows = p.nqkv, R = p.qkv_rows, S = p.qkv_lds_rows, r0 = (int)blockIdx.x * R;
  const int lane = lane_id();
  for (int i = wave_u(); i < S && r0 + i < rows; i += NWAVE) {
    const uint16_t* src = (const uint16_t*)Lw.wqkv + (size_t)(r0 + i) * KK + 8 * lane;
#pragma unroll
    for (int b = 0; b < KK / 512; ++b)
      __builtin_amdgcn_global_load_lds((const MK_G void*)(src + 512 * b),
                                       (__attribute__((address_space(3))) void*)&s.qkvw[i * (KK / 8) + 64 * b], 16, 0, 0);
  }
}

// rows per wave of a workgroup's QKV share beyond the LDS-staged ones (loaded into registers before the wait):
// none for rows of up to 2048 (a share of Qwen3-30B-A3B fits the stage), two for longer rows
template <int KK>
constexpr int qkv_reg_rows() { return KK >= 4096 ? 2 : 0; }

// P1 with the weights in LDS (staged by qkv_to_lds one layer ahead) and, past the stage, in registers (loaded
// before the wait): the same norm prologue, the same dot order.
template <int KK, class Wait>
__device__ __forceinline__ void phase_qkv_lds(const Params& p, int layer, Smem& s, Wait wait) {
  using WR = Bf16Row<KK>;
  constexpr int RR = qkv_reg_rows<KK>();
  const LayerW Lw = layer_w(p, layer);
  const int rows = p.nqkv, R = p.qkv_rows, S = p.qkv_lds_rows, r0 = (int)blockIdx.x * R;
  const int lane = lane_id(), wave = wave_u();
  float* qkv = p.qkv;
  typename WR::Regs Rr[RR > 0 ? RR : 1];
#pragma unroll
  for (int u = 0; u < RR; ++u) {                          // rows S + wave + 8u
    const int i = S + wave + u * NWAVE;
    if (i < R && r0 + i < rows) WR::load(Rr[u], mrow<WR>(Lw.wqkv, (size_t)(r0 + i)), lane);
  }
  if (!wait()) return;
  build_norm_x<KK>(p, p.x, nullptr, Lw.ln1, s);
  if (blockIdx.x == 0 && p.dump_x && layer > p.l0)
    for (int i = threadIdx.x; i < KK; i += NT) st_f(p.dump_x + (size_t)(layer - 1) * KK + i, s.g.xf[i]);
  __builtin_amdgcn_s_waitcnt(0);                          // this wave's rows have landed in LDS (long since)
  for (int i = wave; i < S && r0 + i < rows; i += NWAVE) {
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < KK / 512; ++b) {
      const u32x4 w = s.qkvw[i * (KK / 8) + 64 * b + lane];
      const u32x4 xv = *(const u32x4*)(s.g.xs + 512 * b + lane * 8);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc = __builtin_fmaf(bf_lo(w[j]), bf_lo(xv[j]), acc);
        acc = __builtin_fmaf(bf_hi(w[j]), bf_hi(xv[j]), acc);
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) st_ag(qkv + r0 + i, bfr(acc));
  }
#pragma unroll
  for (int u = 0; u < RR; ++u) {
    const int i = S + wave + u * NWAVE;
    if (i < R && r0 + i < rows) {
      const float acc = WR::dot(Rr[u], s.g.xs, lane);
      if (lane == 0) st_ag(qkv + r0 + i, bfr(acc));
    }
  }
}

// P1: input RMSNorm + fused QKV GEMV (ref_numpy.py:111-115)
template <class WR, class Wait>
__device__ __forceinline__ void phase_qkv(const Params& p, int layer, Smem& s, Wait wait) {
  constexpr int KK = WR::K;
  const LayerW Lw = layer_w(p, layer);
  const bool first = layer == p.l0 && p.do_embed;
  const int rows = p.nqkv;
  float* qkv = p.qkv;
  const uint8_t* W = Lw.wqkv;
  gemv_run<WR, 2>(
      (rows + 1) / 2,
      [&](int g, int i) -> const uint8_t* { const int r = 2 * g + i; return r < rows ? mrow<WR>(W, r) : nullptr; },
      [&](int) { return (const uint16_t*)s.g.xs; },
      [&](int g, const float(&v)[2]) {
        lane_store<2>(v, [&](int i, float val) { const int r = 2 * g + i; if (r < rows) st_ag(qkv + r, bfr(val)); });
      },
      [&]() {
        if (!wait()) return false;
        const uint16_t* xrow = first ? p.embed + (size_t)token_of(p) * KK : nullptr;
        build_norm_x<KK>(p, p.x, xrow, Lw.ln1, s);
        if (blockIdx.x == 0) {
          if (p.dump_x && layer > p.l0)
            for (int i = threadIdx.x; i < KK; i += NT) st_f(p.dump_x + (size_t)(layer - 1) * KK + i, s.g.xf[i]);
          if (layer == p.l0 && p.do_head && threadIdx.x == 0)
            __hip_atomic_store(p.amax, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return true;
      },
      p.nwg, p.trace, s.phase);
}

// P2: per (kv head, 64-position chunk, half of the group's q heads): q/k RMSNorm and neox RoPE of the item's heads
// (ref_numpy.py:116-120), paged KV append by the first half's item of the chunk holding `pos` (:121), then per q
// head the chunk's scores, max, exp, sum and probability-weighted V (:122-129 in chunked form).  The chunk partials
// (a[HD], m, l) go to global memory; the last chunk of a (kv head, half) to arrive merges them in ascending chunk
// order and writes o.
// per-head RMSNorm of (a0, a1) = dims (lane, lane + 64) with weights (w0, w1)
__device__ __forceinline__ void qk_norm(float& a0, float& a1, float w0, float w1, float eps) {
  float acc = __builtin_fmaf(a0, a0, 0.0f);
  acc = __builtin_fmaf(a1, a1, acc);
  acc = wave_sum(acc);
  const float r = 1.0f / __builtin_sqrtf(acc / (float)HDIM + eps);
  a0 = bfr(w0 * bfr(a0 * r));
  a1 = bfr(w1 * bfr(a1 * r));
}

// One attention work item: sequence b (always 0 in single-sequence kernels), kv head g, and CPI consecutive chunks
// cp*CPI, ... of the sequence's positions 0..pos.  Items are numbered sequence by sequence (p.ibase), kv head fastest.
struct AttnItem {
  int b, g, cp, pos;
};
template <int B, int CPI>
__device__ __forceinline__ AttnItem attn_item(const Params& p, int item) {
  int b = 0, r = item;
  if constexpr (B > 1) {
    while (b + 1 < p.B && item >= p.ibase[b + 1]) ++b;
    r = item - p.ibase[b];
  }
  return AttnItem{b, r % p.NKV, r / p.NKV, B > 1 ? p.posb[b] : p.pos};
}

// the single-sequence phase (the batched kernels run phase_attn_b and phase_attn_merge_b)
template <int B, class S, class Wait>
__device__ __forceinline__ void phase_attn(const Params& p, int layer, S& s, Wait wait) {
  static_assert(B == 1, "single-sequence attention");
  constexpr int CPI = decltype(s.a)::cpi;
  const int NKV = p.NKV, NH = p.NH, G = NH / NKV, HD = HDIM, BS = p.BS;
  const int NQKV = (NH + 2 * NKV) * HD;
  // Items (kv head, chunk, half of the kv head's q heads): twice the workgroups of one item per (kv head, chunk),
  // each computing on one wave per SIMD (the score and P.V chains are VALU-bound; with a whole group's heads two
  // waves shared each SIMD), and half of the grid still free to stream the O projection's rows during the phase.
  // Quarters (every workgroup an item at context 1024) left no workgroup to do that and were slower.
  const int HS = (G % 2 == 0) ? 2 : 1, GH = G / HS;
  const int nitems = HS * NKV * ((p.pos / CHUNK + CPI) / CPI);
  const LayerW Lw = layer_w(p, layer);
  const int lane = lane_id(), wave = wave_u();
  // The chunks' cached K and V go straight from HBM into LDS tiles (global_load_lds, 16 bytes per lane); they do
  // not depend on this step, so the first item's copies are issued before the wait.  Wave w copies K dim-groups
  // 2w, 2w+1 (lane = position) and the V position-group w (lane = dim, both halves) of every chunk of the item.
  // The current position is not read from the cache: it is patched into the tiles from the QKV row.
  auto load_kv = [&](int item) {
    const AttnItem it = attn_item<B, CPI>(p, item / HS);
    const int g = it.g, pos = it.pos, n = pos + 1, nch = (n + CHUNK - 1) / CHUNK, fp = pos;
    const int32_t* btab = p.btab + (size_t)it.b * p.nbps;
#pragma unroll
    for (int ci = 0; ci < CPI; ++ci) {
      const int c = it.cp * CPI + ci;
      if (c < nch) {
        const int t0 = c * CHUNK, len = min(CHUNK, n - t0);
        const int t = t0 + lane;
        if (lane < len && t < fp) {
          const int blk = ld_i(btab + t / BS), off = t % BS;
          const uint16_t* kp = Lw.kc + (((size_t)blk * NKV + g) * (HD / 8)) * BS * 8 + off * 8;
#pragma unroll
          for (int jj = 2 * wave; jj < 2 * wave + 2; ++jj)
            __builtin_amdgcn_global_load_lds((const MK_G void*)(kp + (size_t)jj * BS * 8),
                                             (__attribute__((address_space(3))) void*)&s.a.kt[ci][jj][0], 16, 0, 0);
        }
        const int tb = t0 + wave * 8;                     // 8 positions per 16-byte load
        if (tb < t0 + len && tb < fp) {
          const int blk = ld_i(btab + tb / BS), off = tb % BS;
          const uint16_t* vp = Lw.vc + ((size_t)blk * NKV + g) * HD * BS + off;
          __builtin_amdgcn_global_load_lds((const MK_G void*)(vp + (size_t)lane * BS),
                                           (__attribute__((address_space(3))) void*)&s.a.vt[ci][wave][0][0], 16, 0, 0);
          __builtin_amdgcn_global_load_lds((const MK_G void*)(vp + (size_t)(lane + 64) * BS),
                                           (__attribute__((address_space(3))) void*)&s.a.vt[ci][wave][1][0], 16, 0, 0);
        }
      }
    }
  };
  // RoPE factors of the position (ref_numpy.py:76-81 tables)
  const float rc = ld_f(p.rope_cos + (size_t)p.pos * (HD / 2) + lane), rs = ld_f(p.rope_sin + (size_t)p.pos * (HD / 2) + lane);
  const float qn0 = bf2f(ld_u16(Lw.qn + lane)), qn1 = bf2f(ld_u16(Lw.qn + lane + 64));
  const float kn0 = bf2f(ld_u16(Lw.kn + lane)), kn1 = bf2f(ld_u16(Lw.kn + lane + 64));
  if ((int)blockIdx.x < nitems) load_kv(blockIdx.x);
  if (!wait()) return;
  for (int item = blockIdx.x; item < nitems; item += p.nwg) {
    const AttnItem it = attn_item<B, CPI>(p, item / HS);
    const int half = item % HS, h0 = it.g * G + half * GH;   // this item's q heads h0 .. h0 + GH - 1
    const int g = it.g, pos = it.pos, n = pos + 1, nch = (n + CHUNK - 1) / CHUNK;
    const int c0 = it.cp * CPI, nc = min(CPI, nch - c0);   // chunks c0 .. c0 + nc - 1
    const int32_t* btab = p.btab + (size_t)it.b * p.nbps;
    const float* qkv = p.qkv + (size_t)it.b * NQKV;
    float* apart = p.apart + (size_t)it.b * NH * MAX_CHUNKS * PART;
    uint32_t* acnt = p.acnt + (size_t)it.b * NKV * 64;
    float* o = p.o + (size_t)it.b * NH * HD;
    // the current position, when it lies in the item's chunks: [qlo, qhi] is it or empty
    const int qlo = max(pos, c0 * CHUNK), qhi = min(pos, (c0 + nc) * CHUNK - 1);
    if (item != (int)blockIdx.x) load_kv(item);
    // wave j computes head g*G + j (G <= 8, checked by the host): its roped q stays in registers, dims lane (q0)
    // and lane + 64 (q1) (ref_numpy.py:116-120); the score and P.V loops take each dim's or position's value from its
    // lane with v_readlane (wave-uniform operands, no LDS traffic for q or p)
    const int j = wave;
    float q0 = 0.0f, q1 = 0.0f;
    if (j < GH) {
      const float* src = qkv + (size_t)(h0 + j) * HD;
      float a0 = ld_ag(src + lane), a1 = ld_ag(src + lane + 64);
      if (p.qk_norm) qk_norm(a0, a1, qn0, qn1, p.eps);
      q0 = bfr(bfr(a0 * rc) + bfr(-a1 * rs));
      q1 = bfr(bfr(a1 * rc) + bfr(a0 * rs));
    }
    // k (normed and roped) and v of the current position come from its QKV row; wave NWAVE-1 takes it
    constexpr int PQ = 1;
    float kn[PQ][2], vn[PQ][2];
#pragma unroll
    for (int u = 0; u < PQ; ++u) {
      const int q = qlo + (NWAVE - 1 - wave) + u * NWAVE;
      if (q <= qhi) {
        const float* row = p.qkv + (size_t)(it.b - (pos - q)) * NQKV;
        const float* ks = row + (size_t)(NH + g) * HD;
        const float* vs = row + (size_t)(NH + NKV + g) * HD;
        float a0 = ld_ag(ks + lane), a1 = ld_ag(ks + lane + 64);
        vn[u][0] = ld_ag(vs + lane);
        vn[u][1] = ld_ag(vs + lane + 64);
        float cq = rc, sq = rs;                           // RoPE factors of position q
        if (q != pos) {
          cq = ld_f(p.rope_cos + (size_t)q * (HD / 2) + lane);
          sq = ld_f(p.rope_sin + (size_t)q * (HD / 2) + lane);
        }
        if (p.qk_norm) qk_norm(a0, a1, kn0, kn1, p.eps);
        kn[u][0] = bfr(bfr(a0 * cq) + bfr(-a1 * sq));
        kn[u][1] = bfr(bfr(a1 * cq) + bfr(a0 * sq));
      }
    }
    __builtin_amdgcn_s_waitcnt(0);                        // this wave's tile copies have landed in LDS
    __syncthreads();
#pragma unroll
    for (int u = 0; u < PQ; ++u) {                        // the new positions' bf16 k, v into the tiles
      const int q = qlo + (NWAVE - 1 - wave) + u * NWAVE;
      if (q <= qhi) {
        const int ci = q / CHUNK - c0, tn = q % CHUNK;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int d = lane + 64 * h;
          ((uint16_t*)&s.a.kt[ci][d / 8][tn])[d % 8] = f2bf(kn[u][h]);
          ((uint16_t*)&s.a.vt[ci][tn / 8][h][lane])[tn % 8] = f2bf(vn[u][h]);
        }
        if (q == pos && half == 0) {                      // paged append (:121): K [blk][NKV][HD/8][BS][8], V [blk][NKV][HD][BS]
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
    auto bcast = [](float v, int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l)); };
    // per chunk: scores (:126): lane = position t0 + lane; s_t = (q . k_t in ascending d) * scale; the chunk max m;
    // p_t = exp(s_t - m) in lane t.  Then V (:127-128): lanes = dims (lane, lane + 64); a = sum_t p_t v_t[d] and
    // l = sum_t p_t, ascending t, from one 16-byte read per dim half (8 positions of this lane's dim).  Full chunks
    // take the loop without position tests; only a head's last chunk is partial.
    // (the V reads run one 8-position group ahead of the chains)
    auto pv = [&](int ci, int len, float pr, auto full, float& a0, float& a1, float& l) {
      u32x4 wn0 = s.a.vt[ci][0][0][lane], wn1 = s.a.vt[ci][0][1][lane];
#pragma unroll
      for (int hb = 0; hb < CHUNK / 8; ++hb) {
        const u32x4 w0 = wn0, w1 = wn1;
        if (hb + 1 < CHUNK / 8 && (decltype(full)::value || (hb + 1) * 8 < len)) {
          wn0 = s.a.vt[ci][hb + 1][0][lane];
          wn1 = s.a.vt[ci][hb + 1][1][lane];
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (decltype(full)::value || hb * 8 + e < len) {
            const float pt = bcast(pr, hb * 8 + e);
            const float v0 = (e & 1) ? bf_hi(w0[e >> 1]) : bf_lo(w0[e >> 1]);
            const float v1 = (e & 1) ? bf_hi(w1[e >> 1]) : bf_lo(w1[e >> 1]);
            a0 = __builtin_fmaf(pt, v0, a0);
            a1 = __builtin_fmaf(pt, v1, a1);
            l = l + pt;
          }
        }
      }
    };
    if (j < GH) {
#pragma unroll
      for (int ci = 0; ci < CPI; ++ci) {
        if (ci < nc) {
          const int c = c0 + ci, len = min(CHUNK, n - c * CHUNK);
          const bool valid = lane < len;
          // the K reads run two 8-dim groups ahead of the chain
          float acc = 0.0f;
          u32x4 kr[HDIM / 8];
          kr[0] = s.a.kt[ci][0][lane];
          kr[1] = s.a.kt[ci][1][lane];
#pragma unroll
          for (int jj = 0; jj < HDIM / 8; ++jj) {
            if (jj + 2 < HDIM / 8) kr[jj + 2] = s.a.kt[ci][jj + 2][lane];
            const u32x4 kw = kr[jj];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int d = 8 * jj + 2 * e;
              acc = __builtin_fmaf(bcast(d < 64 ? q0 : q1, d & 63), bf_lo(kw[e]), acc);
              acc = __builtin_fmaf(bcast(d + 1 < 64 ? q0 : q1, (d + 1) & 63), bf_hi(kw[e]), acc);
            }
          }
          const float sc = valid ? acc * p.attn_scale : -__builtin_huge_valf();
          const float m = wave_max(sc);
          const float pr = valid ? expf_mk(sc - m) : 0.0f;
          float a0 = 0.0f, a1 = 0.0f, l = 0.0f;
          if (len == CHUNK) pv(ci, len, pr, std::true_type{}, a0, a1, l);
          else pv(ci, len, pr, std::false_type{}, a0, a1, l);
          float* part = apart + ((size_t)(h0 + j) * MAX_CHUNKS + c) * PART;
          st_ag(part + lane, a0);
          st_ag(part + lane + 64, a1);
          if (lane == 0) { st_ag(part + HD, m); st_ag(part + HD + 1, l); }
        }
      }
    }
    if (p.trace && threadIdx.x == 0)                      // slot 2 of the attention phase: chunk partials issued
      *(MK_G uint64_t*)(p.trace + ((size_t)s.phase * p.nwg + blockIdx.x) * 3 + 2) = __builtin_amdgcn_s_memrealtime();
    // the last item of kv head g to arrive merges: M = max m_c, w_c = exp(m_c - M), L = sum w_c l_c,
    // A[d] = sum w_c a_c[d] (ascending c), o = bfr(A / L)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      const uint32_t old = __hip_atomic_fetch_add(acnt + 64 * (g * HS + half), (uint32_t)nc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s.last = (old + (uint32_t)nc == (uint32_t)nch);
    }
    __syncthreads();
    if (s.last) {
      for (int j = wave; j < GH; j += NWAVE) {
        const float* part = apart + (size_t)(h0 + j) * MAX_CHUNKS * PART;
        // lane cc holds chunks cc and cc + 64's (m, l); the chunk weights go through LDS for the ordered sums.  The
        // first MB chunks' a[] are loaded together with (m, l) (they do not depend on the maximum): one round trip.
        constexpr int MB = 18;
        float av0[MB], av1[MB];
        auto load_a = [&](int cb) {
#pragma unroll
          for (int u = 0; u < MB; ++u) {
            const int c = min(cb + u, nch - 1);             // past the last chunk: a repeat, never used
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
        s.a.p[j][lane] = lane < nch ? expf_mk(mloc - M) : 0.0f;
        s.a.p[j][64 + lane] = lane + 64 < nch ? expf_mk(mhi - M) : 0.0f;
        s.a.p[j][MAX_CHUNKS + lane] = lloc;
        s.a.p[j][MAX_CHUNKS + 64 + lane] = lhi;
        float Ls = 0.0f, A0 = 0.0f, A1 = 0.0f;
        for (int cb = 0; cb < nch; cb += MB) {
          if (cb > 0) load_a(cb);
#pragma unroll
          for (int u = 0; u < MB; ++u)
            if (cb + u < nch) {
              const float wc = s.a.p[j][cb + u];
              Ls = __builtin_fmaf(wc, s.a.p[j][MAX_CHUNKS + cb + u], Ls);
              A0 = __builtin_fmaf(wc, av0[u], A0);
              A1 = __builtin_fmaf(wc, av1[u], A1);
            }
        }
        st_ag(o + (size_t)(h0 + j) * HD + lane, bfr(A0 / Ls));
        st_ag(o + (size_t)(h0 + j) * HD + lane + 64, bfr(A1 / Ls));
      }
      if (threadIdx.x == 0) __hip_atomic_store(acnt + 64 * (g * HS + half), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
  }
}

// P3: O projection and residual (ref_numpy.py:130): x = bfr(x + bfr(Wo . o)); the residual is read into LDS in
// the prologue together with o, so the epilogue does not wait on memory.  HQ > 0 (persistent kernel): the next
// layer's QKV rows of this workgroup start streaming into LDS right behind the O rows; the attention and router
// phases around it leave the memory system room for them (a dense model's O phase absorbs them less well, yet
// better than its gate/up phase: 3.140 against 3.176 ms/token for Qwen3-8B).
template <class WR, class Wait, int HQ = 0>
__device__ __forceinline__ void phase_oproj(const Params& p, int layer, Smem& s, Wait wait) {
  constexpr int KK = WR::K;
  const LayerW Lw = layer_w(p, layer);
  const int H = p.H;
  const bool first = layer == p.l0 && p.do_embed;
  float* x = p.x;
  const uint8_t* W = Lw.wo;
  gemv_run<WR, 1>(
      H,
      [&](int g, int) -> const uint8_t* { return mrow<WR>(W, g); },
      [&](int) { return (const uint16_t*)s.g.xs; },
      [&](int g, const float(&v)[1]) {
        if (lane_id() == 0) st_ag(x + g, bfr(s.g.xf[g] + bfr(v[0])));
      },
      [&]() {
        if constexpr (HQ > 0)
          if (p.qkv_rows > 0 && layer + 1 < p.l1) qkv_to_lds<HQ>(p, layer + 1, s);
        if (!wait()) return false;
        load_vec_perm<KK, 1>(p.o, 1, s.g.xs);
        load_residual(p, first, first ? token_of(p) : 0, s.g.xf);
        __syncthreads();
        return true;
      },
      p.nwg, p.trace, s.phase);
}

// P4: post-attention RMSNorm + router GEMV (ref_numpy.py:131-134)
template <int KK, class Wait>
__device__ __forceinline__ void phase_router(const Params& p, int layer, Smem& s, Wait wait) {
  using WR = Bf16Row<KK>;                                 // the router stays bf16 in every weight type
  const LayerW Lw = layer_w(p, layer);
  const int E = p.E;
  float* lg = p.logits;
  const uint8_t* W = Lw.wr;
  gemv_run<WR, 1>(
      E,
      [&](int g, int) -> const uint8_t* { return mrow<WR>(W, g); },
      [&](int) { return (const uint16_t*)s.g.xs; },
      [&](int g, const float(&v)[1]) { if (lane_id() == 0) st_ag(lg + g, bfr(v[0])); },
      [&]() {
        if (!wait()) return false;
        build_norm_x<KK>(p, p.x, nullptr, Lw.ln2, s);
        return true;
      },
      p.nwg, p.trace, s.phase);
}

// softmax top-k over the router logits (ref_numpy.py:135-140).  Every wave computes it on its own, in registers:
// fp32 probabilities (max, exp, the dot-order sum, divide), then K rounds of "largest probability, lowest id
// first" (a wave max, then the lowest lane of the first 64-expert word whose ballot holds it); a chosen expert
// drops to -2, below every probability and below the -1 of absent experts.  The chosen probabilities are
// renormalised in slot order and rounded to bf16; `order` lists the slots by ascending expert id (the index_add_
// order of the combine).  Results land in the wave's private LDS row s.ids/wts/order[wave].
template <int EC>
struct RouteLogits {
  static constexpr int NW = ((EC > 0 ? EC : MAX_E) + 63) / 64;
  float v[NW];
};
// lane l's logits of experts l, l + 64, ... (agent-scope: written by the router phase); absent experts -inf
template <int EC = 0>
__device__ __forceinline__ void route_load(const Params& p, const float* logits, RouteLogits<EC>& r) {
  const int E = EC > 0 ? EC : p.E, lane = lane_id();
#pragma unroll
  for (int w = 0; w < RouteLogits<EC>::NW; ++w) {
    const int e = lane + 64 * w;
    r.v[w] = e < E ? ld_ag(logits + e) : -__builtin_huge_valf();
  }
}
template <int EC = 0>
__device__ __forceinline__ void route_topk_from(const Params& p, RouteLogits<EC> r, int32_t* ids_out, float* wts_out,
                                                int32_t* order_out) {
  constexpr int NW = RouteLogits<EC>::NW;
  const int E = EC > 0 ? EC : p.E, K = p.TOPK;
  const int lane = lane_id();
  float (&pv)[NW] = r.v;
  float m = pv[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) m = fmaxf(m, pv[w]);
  m = wave_max(m);
  float acc = 0.0f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int e = lane + 64 * w;
    pv[w] = e < E ? expf_mk(pv[w] - m) : 0.0f;
    if (e < E) acc = acc + pv[w];
  }
  const float S = wave_sum(acc);
#pragma unroll
  for (int w = 0; w < NW; ++w) pv[w] = lane + 64 * w < E ? pv[w] / S : -1.0f;
  int ids[MAX_TOPK];
  float pk[MAX_TOPK];
  float sel = 0.0f;
#pragma unroll
  for (int k = 0; k < MAX_TOPK; ++k) {
    ids[k] = 0;
    pk[k] = 0.0f;
    if (k < K) {
      float b = pv[0];
#pragma unroll
      for (int w = 1; w < NW; ++w) b = fmaxf(b, pv[w]);
      b = wave_max(b);
      int id = -1;
#pragma unroll
      for (int w = NW - 1; w >= 0; --w) {
        const uint64_t hit = __ballot(pv[w] == b);
        if (hit) id = 64 * w + __builtin_ctzll(hit);
      }
#pragma unroll
      for (int w = 0; w < NW; ++w)
        if (lane + 64 * w == id) pv[w] = -2.0f;
      ids[k] = id < 0 ? 0 : id;                           // only NaN logits leave no hit; keep the index in range
      pk[k] = b;
      sel = sel + b;
    }
  }
  if (lane < MAX_TOPK) {
    int id = 0, before = 0;
    float wk = 0.0f;
#pragma unroll
    for (int k = 0; k < MAX_TOPK; ++k)
      if (k == lane) { id = ids[k]; wk = pk[k]; }
#pragma unroll
    for (int k = 0; k < MAX_TOPK; ++k)
      if (k < K && ids[k] < id) ++before;
    if (lane < K) {
      ids_out[lane] = id;
      // Qwen3: bf16 weights, renormalised (ref_numpy.py:138-140); DeepSeek-V2: fp32 probability times
      // routed_scaling_factor, or renormalised with a 1e-20 guard (reference_decode.py:271-278)
      if (p.arch == ETXMK_ARCH_DSV2) wts_out[lane] = p.norm_topk ? wk / (sel + 1e-20f) : wk * p.routed_scale;
      else wts_out[lane] = bfr(p.norm_topk ? wk / sel : wk);
      if (order_out) order_out[before] = lane;
    }
  }
}
template <int EC = 0>
__device__ __forceinline__ void route_topk_into(const Params& p, const float* logits, int32_t* ids_out, float* wts_out,
                                                int32_t* order_out) {
  RouteLogits<EC> r;
  route_load<EC>(p, logits, r);
  route_topk_from<EC>(p, r, ids_out, wts_out, order_out);
}
// every wave routes on its own from the logits, which one wave reads (agent-scope) into LDS for the workgroup:
// the grid's reads of the one logits row are one per workgroup, not one per wave
template <int EC = 0>
__device__ __forceinline__ void route_topk(const Params& p, Smem& s) {
  const int wave = wave_u(), lane = lane_id(), E = EC > 0 ? EC : p.E;
  if (wave == 0) {
    RouteLogits<EC> r;
    route_load<EC>(p, p.logits, r);
#pragma unroll
    for (int w = 0; w < RouteLogits<EC>::NW; ++w)
      if (lane + 64 * w < E) s.lg[lane + 64 * w] = r.v[w];
  }
  __syncthreads();
  RouteLogits<EC> r;
#pragma unroll
  for (int w = 0; w < RouteLogits<EC>::NW; ++w) r.v[w] = lane + 64 * w < E ? s.lg[lane + 64 * w] : -__builtin_huge_valf();
  route_topk_from<EC>(p, r, s.ids[wave], s.wts[wave], s.order[wave]);
}

// P5: experts gate/up + SiLU*up for the top-k slots (ref_numpy.py:142-145).  The normed input depends only on x
// (final since the O projection), so it is built before the wait; the routing needs this phase's inputs.
template <class WR, class Wait, int EC = 0>
__device__ __forceinline__ void phase_expert_up(const Params& p, int layer, Smem& s, Wait wait) {
  constexpr int KK = WR::K;
  const LayerW Lw = layer_w(p, layer);
  const int MI = p.MI, KT = p.TOPK;
  float* hb = p.hbuf;
  const uint8_t* W = Lw.w13;
  build_norm_x<KK>(p, p.x, nullptr, Lw.ln2, s);
  if (!wait()) return;
  route_topk<EC>(p, s);
  if (blockIdx.x == 0 && threadIdx.x < 64) {
    const int t = threadIdx.x;
    if (p.dump_ids && t < KT) st_i(p.dump_ids + (size_t)layer * KT + t, s.ids[0][t]);
    if (p.dump_wts && t < KT) st_f(p.dump_wts + (size_t)layer * KT + t, s.wts[0][t]);
    if (p.dump_logits)
      for (int e = t; e < p.E; e += 64) st_f(p.dump_logits + (size_t)layer * p.E + e, ld_ag(p.logits + e));
  }
  gemv_run<WR, 2>(
      KT * MI,
      [&](int g, int i) -> const uint8_t* {
        const int slot = g / MI, jj = g - slot * MI;
        return mrow<WR>(W, (size_t)s.ids[wave_u()][slot] * 2 * MI + 2 * jj + i);
      },
      [&](int) { return (const uint16_t*)s.g.xs; },
      [&](int g, const float(&v)[2]) {
        if (lane_id() == 0) st_ag(hb + g, bfr(bfr(silu(bfr(v[0]))) * bfr(v[1])));
      },
      [&]() { return true; }, p.nwg, p.trace, s.phase);
}

// P6: expert down, routing weight, combine in ascending expert id, residual (ref_numpy.py:146-148).  The routing
// comes from the router logits, final since two barriers ago, so the weights stream before the wait.
template <class WR, class Wait, bool ROUTED = false>
__device__ __forceinline__ void phase_expert_down(const Params& p, int layer, Smem& s, Wait wait) {
  constexpr int KK = WR::K;
  const LayerW Lw = layer_w(p, layer);
  const int H = p.H, KT = p.TOPK;
  if constexpr (!ROUTED) route_topk(p, s);                 // the persistent kernel keeps expert_up's routing in LDS
  float* x = p.x;
  const uint8_t* W = Lw.w2;
  gemv_run<WR, MAX_TOPK>(
      H,
      [&](int g, int i) -> const uint8_t* { return i < KT ? mrow<WR>(W, (size_t)s.ids[wave_u()][i] * H + g) : nullptr; },
      [&](int i) { return (const uint16_t*)(s.g.xs + (size_t)i * KK); },
      [&](int g, const float(&v)[MAX_TOPK]) {
        if (lane_id() == 0) {
          float y[MAX_TOPK];
#pragma unroll
          for (int i = 0; i < MAX_TOPK; ++i) y[i] = i < KT ? bfr(bfr(v[i]) * s.wts[wave_u()][i]) : 0.0f;
          float acc = 0.0f;
          for (int k = 0; k < KT; ++k) {
            const int o = s.order[wave_u()][k];
            float yk = 0.0f;
#pragma unroll
            for (int i = 0; i < MAX_TOPK; ++i) yk = (o == i) ? y[i] : yk;
            acc = bfr(acc + yk);
          }
          st_ag(x + g, bfr(s.g.xf[g] + acc));
        }
      },
      [&]() {
        if (!wait()) return false;
        load_vec_perm<KK, MAX_TOPK>(p.hbuf, KT, s.g.xs);
        load_x(p.x, p.H, s.g.xf);
        __syncthreads();
        return true;
      },
      p.nwg, p.trace, s.phase);
}

// dense MLP (ref_numpy.py:149-152): P4' gate/up + SiLU*up, P5' down + residual
template <class WR, class Wait>
__device__ __forceinline__ void phase_gateup(const Params& p, int layer, Smem& s, Wait wait) {
  constexpr int KK = WR::K;
  const LayerW Lw = layer_w(p, layer);
  float* hb = p.hbuf;
  const uint8_t* W = Lw.wgu;
  gemv_run<WR, 2>(
      p.I,
      [&](int g, int i) -> const uint8_t* { return mrow<WR>(W, (size_t)2 * g + i); },
      [&](int) { return (const uint16_t*)s.g.xs; },
      [&](int g, const float(&v)[2]) {
        if (lane_id() == 0) st_ag(hb + g, bfr(bfr(silu(bfr(v[0]))) * bfr(v[1])));
      },
      [&]() {
        if (!wait()) return false;
        build_norm_x<KK>(p, p.x, nullptr, Lw.ln2, s);
        return true;
      },
      p.nwg, p.trace, s.phase);
}

template <class WR, class Wait>
__device__ __forceinline__ void phase_down(const Params& p, int layer, Smem& s, Wait wait) {
  constexpr int KK = WR::K;
  const LayerW Lw = layer_w(p, layer);
  float* x = p.x;
  const uint8_t* W = Lw.wd;
  gemv_run<WR, 1>(
      p.H,
      [&](int g, int) -> const uint8_t* { return mrow<WR>(W, g); },
      [&](int) { return (const uint16_t*)s.g.xs; },
      [&](int g, const float(&v)[1]) {
        if (lane_id() == 0) st_ag(x + g, bfr(s.g.xf[g] + bfr(v[0])));
      },
      [&]() {
        if (!wait()) return false;
        load_vec_perm<KK, 1>(p.hbuf, 1, s.g.xs);
        load_x(p.x, p.H, s.g.xf);
        __syncthreads();
        return true;
      },
      p.nwg, p.trace, s.phase);
}

// P7: final norm + lm_head + per-wave argmax folded into one 64-bit key (ref_numpy.py:155-158; first maximum wins)
__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {
  if (v == 0.0f) v = 0.0f;                                // -0 and +0 compare equal, as in torch.argmax
  const uint32_t u = f2bits(v);
  const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)idx);
}

template <int KK, class Wait>
__device__ __forceinline__ void phase_head(const Params& p, Smem& s, Wait wait) {
  using WR = Bf16Row<KK>;                                 // lm_head stays bf16 in every weight type
  const int V = p.V;
  const uint8_t* W = (const uint8_t*)p.lm_head;
  uint64_t best = 0;
  bool ran = false;
  ran = gemv_run<WR, 2>(
      (V + 1) / 2,
      [&](int g, int i) -> const uint8_t* { const int r = 2 * g + i; return r < V ? mrow<WR>(W, r) : nullptr; },
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
      },
      [&]() {
        if (!wait()) return false;
        build_norm_x<KK>(p, p.x, nullptr, p.final_norm, s);
        if (blockIdx.x == 0 && p.dump_x)
          for (int i = threadIdx.x; i < KK; i += NT) st_f(p.dump_x + (size_t)(p.l1 - 1) * KK + i, s.g.xf[i]);
        return true;
      },
      p.nwg, p.trace, s.phase);
  if (ran && lane_id() == 0 && best) __hip_atomic_fetch_max(p.amax, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <class Wait>
__device__ __forceinline__ void phase_token(const Params& p, Wait wait) {
  if (!wait()) return;
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

// runtime row-length dispatch (unfused per-phase kernels)
template <class Wait>
__device__ __forceinline__ void phase_qkv_any(const Params& p, int layer, Smem& s, Wait wait) {
  dispatch_k<MK_K_HIDDEN>(p.H, [&](auto kc_) { phase_qkv<Bf16Row<decltype(kc_)::value>>(p, layer, s, wait); });
}
template <class Wait>
__device__ __forceinline__ void phase_oproj_any(const Params& p, int layer, Smem& s, Wait wait) {
  dispatch_k<MK_K_ATTN>(p.NH * p.HD, [&](auto kc_) { phase_oproj<Bf16Row<decltype(kc_)::value>>(p, layer, s, wait); });
}
template <class Wait>
__device__ __forceinline__ void phase_router_any(const Params& p, int layer, Smem& s, Wait wait) {
  dispatch_k<MK_K_HIDDEN>(p.H, [&](auto kc_) { phase_router<decltype(kc_)::value>(p, layer, s, wait); });
}
template <class Wait>
__device__ __forceinline__ void phase_expert_up_any(const Params& p, int layer, Smem& s, Wait wait) {
  dispatch_k<MK_K_HIDDEN>(p.H, [&](auto kc_) { phase_expert_up<Bf16Row<decltype(kc_)::value>>(p, layer, s, wait); });
}
template <class Wait>
__device__ __forceinline__ void phase_expert_down_any(const Params& p, int layer, Smem& s, Wait wait) {
  dispatch_k<MK_K_MOE>(p.MI, [&](auto kc_) { phase_expert_down<Bf16Row<decltype(kc_)::value>>(p, layer, s, wait); });
}
template <class Wait>
__device__ __forceinline__ void phase_gateup_any(const Params& p, int layer, Smem& s, Wait wait) {
  dispatch_k<MK_K_HIDDEN>(p.H, [&](auto kc_) { phase_gateup<Bf16Row<decltype(kc_)::value>>(p, layer, s, wait); });
}
template <class Wait>
__device__ __forceinline__ void phase_down_any(const Params& p, int layer, Smem& s, Wait wait) {
  dispatch_k<MK_K_INTER>(p.I, [&](auto kc_) { phase_down<Bf16Row<decltype(kc_)::value>>(p, layer, s, wait); });
}
template <class Wait>
__device__ __forceinline__ void phase_head_any(const Params& p, Smem& s, Wait wait) {
  dispatch_k<MK_K_HIDDEN>(p.H, [&](auto kc_) { phase_head<decltype(kc_)::value>(p, s, wait); });
}

// ---------------------------------------------------------------- kernels
enum Phase { PH_QKV = 0, PH_ATTN, PH_OPROJ, PH_ROUTER, PH_EXPUP, PH_EXPDN, PH_GATEUP, PH_DOWN, PH_HEAD, PH_TOKEN };

// The persistent kernel, instantiated per model shape: hidden size H, attention width KA = NH*HD, the MLP row
// length KM (the expert intermediate for MoE, the dense intermediate otherwise) and the weight type (FP8: the
// QKV, O and MLP matrices in Fp8Row format).
template <int H, int KA, int KM, bool MOE, int EC, bool FP8>
__device__ __forceinline__ void fused_body(const Params& p) {
  __shared__ Smem s;
  if (threadIdx.x == 0) s.abort = 0;
  __syncthreads();
  int k = 0;                                              // arrivals so far in this launch
  auto wait = [&]() { return grid_wait(p, k, s); };
  // per-phase timeline (ETX_TRACE, etx/codegen/kernel.py:346-347): 100 MHz s_memrealtime stamps of every
  // workgroup when its wait for the phase's inputs returns and when it arrives after the phase
  if (p.trace && threadIdx.x == 0) *(MK_G uint64_t*)(p.trace + (size_t)blockIdx.x * 3) = __builtin_amdgcn_s_memrealtime();
  s.phase = 0;
  for (int layer = p.l0; layer < p.l1; ++layer) {
    if constexpr (!FP8) {
      if (p.qkv_rows > 0 && layer > p.l0) phase_qkv_lds<H>(p, layer, s, wait);
      else phase_qkv<Bf16Row<H>>(p, layer, s, wait);
    } else {
      phase_qkv<Fp8Row<H>>(p, layer, s, wait);
    }
    if (s.abort) return;
    grid_arrive(p, k, s);
    phase_attn<1>(p, layer, s, wait);
    if (s.abort) return;
    grid_arrive(p, k, s);
    phase_oproj<RowOf<FP8, KA>, decltype(wait), (!FP8 && H % 512 == 0 ? H : 0)>(p, layer, s, wait);
    if (s.abort) return;
    grid_arrive(p, k, s);
    if constexpr (MOE) {
      phase_router<H>(p, layer, s, wait);
      if (s.abort) return;
      grid_arrive(p, k, s);
      phase_expert_up<RowOf<FP8, H>, decltype(wait), EC>(p, layer, s, wait);
      if (s.abort) return;
      grid_arrive(p, k, s);
      phase_expert_down<RowOf<FP8, KM>, decltype(wait), true>(p, layer, s, wait);
      if (s.abort) return;
      grid_arrive(p, k, s);
    } else {
      phase_gateup<RowOf<FP8, H>>(p, layer, s, wait);
      if (s.abort) return;
      grid_arrive(p, k, s);
      phase_down<RowOf<FP8, KM>>(p, layer, s, wait);
      if (s.abort) return;
      grid_arrive(p, k, s);
    }
  }
  if (p.do_head) {
    phase_head<H>(p, s, wait);
    if (s.abort) return;
    grid_arrive(p, k, s);
    phase_token(p, wait);
  }
}

// Shapes with a persistent kernel: name, H, KA, KM, MoE, E, fp8 weights (the host picks by the same fields).  Each
// list is instantiated by its own translation unit (mk_fused_bf16.hip, mk_fused_fp8.hip), so they compile in
// parallel; the host declares them all (MK_FUSED_DECL).
#define MK_FUSED_SHAPES_BF16(X)                                                \
  X(etxmk_fused_h2048_a4096_moe768_e128, 2048, 4096, 768, true, 128, false)   \
  X(etxmk_fused_h4096_a4096_mlp12288, 4096, 4096, 12288, false, 0, false)     \
  X(etxmk_fused_h512_a512_moe256_e16, 512, 512, 256, true, 16, false)         \
  X(etxmk_fused_h512_a512_mlp1024, 512, 512, 1024, false, 0, false)
#define MK_FUSED_SHAPES_FP8(X)                                                 \
  X(etxmk_fused_fp8_h2048_a4096_moe768_e128, 2048, 4096, 768, true, 128, true) \
  X(etxmk_fused_fp8_h512_a512_moe256_e16, 512, 512, 256, true, 16, true)       \
  X(etxmk_fused_fp8_h512_a512_mlp1024, 512, 512, 1024, false, 0, true)
#define MK_FUSED_KERNEL(name, H, KA, KM, MOE, EC, FP8) \
  extern "C" __global__ void __launch_bounds__(NT, 1) name(Params p) { fused_body<H, KA, KM, MOE, EC, FP8>(p); }
#define MK_FUSED_DECL(name, H, KA, KM, MOE, EC, FP8) extern "C" __global__ void __launch_bounds__(NT, 1) name(Params p);

// unfused mode: one kernel per phase, same device functions (named per phase so profiles separate them; bf16
// weights; instantiated by the host translation unit)
struct NoWait {
  __device__ bool operator()() const { return true; }
};
#define MK_PHASE_KERNEL(name, CALL)                                                   \
  extern "C" __global__ void __launch_bounds__(NT, 1) name(Params p, int layer) { \
    __shared__ Smem s;                                                            \
    if (threadIdx.x == 0) s.abort = 0;                                            \
    __syncthreads();                                                              \
    CALL;                                                                         \
  }

}  // namespace mk
