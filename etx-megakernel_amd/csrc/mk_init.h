#pragma once
// Weight and cache initialisation kernels of the host translation unit: the seeded generator, layout packing, fp8
// quantisation and the seeded KV fill.  None of them runs inside a decode step.
#include "mk_device.h"

namespace mk {

// n_t consecutive tensors of rows x cols (experts of one layer); element (r, k) of tensor e is number r*lcols+k
// of stream sid0 + e for k < lcols (the logical row length) and zero in the pads [lcols, cols); stored at its
// lane-permuted position when perm != 0.
extern "C" __global__ void etxmk_gen_weights(uint16_t* dst, uint64_t seed, uint64_t sid0, int n_t, int rows, int cols,
                                             int lcols, int perm, float scale) {
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
      out[u] = k < lcols ? f2bf(scale * normal_at(key, (uint64_t)r * lcols + k)) : (uint16_t)0;
    }
    *(u32x4*)(dst + q) = *(const u32x4*)out;
  }
}

extern "C" __global__ void etxmk_fill_u16(uint16_t* dst, size_t n, uint16_t v) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) dst[i] = v;
}

// natural rows of lcols bf16 -> lane-permuted rows of cols (pads zero)
extern "C" __global__ void etxmk_pack_rows(uint16_t* dst, const uint16_t* src, int rows, int cols, int lcols) {
  const size_t total = (size_t)rows * cols;
  for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total; q += (size_t)gridDim.x * blockDim.x) {
    const int r = (int)(q / cols), p = (int)(q - (size_t)r * cols);
    const int k = perm_logical(p, cols);
    dst[q] = k < lcols ? src[(size_t)r * lcols + k] : (uint16_t)0;
  }
}

// DeepSeek-V2 kv_b_proj ([NH*(nope + vh)][kvl] natural: per head nope W_UK rows, then vh W_UV rows) stored as
// W_UK^T [NH][kvl][nope] (lane-permuted rows of nope) followed by W_UV [NH*vh][kvl] (lane-permuted rows of kvl).
// Values from src (natural rows) or, when src is null, element (r, k) of the natural tensor is number r*kvl + k
// of stream sid.
extern "C" __global__ void etxmk_pack_kvb(uint16_t* dst, const uint16_t* src, uint64_t seed, uint64_t sid, int NH,
                                          int nope, int vh, int kvl, float scale) {
  const size_t n_uk = (size_t)NH * kvl * nope, total = (size_t)NH * (nope + vh) * kvl;
  const uint64_t key = stream_key(seed, sid);
  for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total; q += (size_t)gridDim.x * blockDim.x) {
    size_t r, k;                                          // natural (row, column) of stored element q
    if (q < n_uk) {
      const size_t row = q / nope;                        // W_UK^T row (h, i)
      const int h = (int)(row / kvl), i = (int)(row % kvl), d = perm_logical((int)(q % nope), nope);
      r = (size_t)h * (nope + vh) + d;
      k = i;
    } else {
      const size_t q2 = q - n_uk, row = q2 / kvl;         // W_UV row (h, d)
      const int h = (int)(row / vh), d = (int)(row % vh), i = perm_logical((int)(q2 % kvl), kvl);
      r = (size_t)h * (nope + vh) + nope + d;
      k = i;
    }
    dst[q] = src ? src[r * kvl + k] : f2bf(scale * normal_at(key, (uint64_t)(r * kvl + k)));
  }
}

// latent cache positions [0, npos) of one sequence: element (t, i) is number t*CD + i of the layer's stream, stored
// at [block][i / 8][block_size][i % 8]
extern "C" __global__ void etxmk_gen_latent(uint16_t* kc, const int32_t* btab, uint64_t key, int npos, int CD, int BS) {
  const size_t total = (size_t)npos * CD;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int d = (int)(i % CD), t = (int)(i / CD);
    const int blk = btab[t / BS], off = t % BS;
    kc[(((size_t)blk * (CD / 8) + d / 8) * BS + off) * 8 + d % 8] = f2bf(normal_at(key, i));
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

// OCP e4m3 ("fn": no infinities, max 448) of f, rounded to nearest even and saturated at +-448; below 2^-6 the
// subnormal grid of 2^-9.  The same integer steps as the CPU oracle's f32_to_e4m3.
__device__ __forceinline__ uint8_t f32_to_e4m3(float f) {
  const uint32_t u = f2bits(f);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80);
  const uint32_t a = u & 0x7FFFFFFFu;
  const float af = bits2f(a);
  if (af != af || af >= 448.0f) return (uint8_t)(sign | 0x7E);
  if (af < 0.015625f) return (uint8_t)(sign | (uint8_t)__builtin_rintf(af * 512.0f));
  int e = (int)(a >> 23) - 127;
  uint32_t qm = (a >> 20) & 7, rem = a & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (qm & 1))) ++qm;
  if (qm == 8) { qm = 0; ++e; }
  if (e > 8 || (e == 8 && qm > 6)) return (uint8_t)(sign | 0x7E);
  return (uint8_t)(sign | (uint8_t)((e + 7) << 3) | (uint8_t)qm);
}

// fp8 rows (Fp8Row format: K codes, the fp32 scale, 12 zero bytes) of n_t consecutive tensors of rows x cols, one
// wave per row: s = amax / 448, q = e4m3(w / s).  The bf16 values come from src (natural rows, one tensor) or, when
// src is null, from the seeded generator (tensor e is stream sid0 + e, element (r, k) number r*cols + k).
extern "C" __global__ void etxmk_quant_rows(uint8_t* dst, const uint16_t* src, uint64_t seed, uint64_t sid0, int n_t,
                                            int rows, int cols, float scale) {
  const int lane = threadIdx.x & 63, wpb = blockDim.x / 64;
  const size_t nrows = (size_t)n_t * rows, stride = (size_t)cols + 16;
  for (size_t gr = (size_t)blockIdx.x * wpb + threadIdx.x / 64; gr < nrows; gr += (size_t)gridDim.x * wpb) {
    const int e = (int)(gr / rows), r = (int)(gr - (size_t)e * rows);
    const uint64_t key = stream_key(seed, sid0 + (uint64_t)e);
    auto val = [&](int k) -> float {
      return src ? bf2f(src[gr * cols + k]) : bf2f(f2bf(scale * normal_at(key, (uint64_t)r * cols + k)));
    };
    float amax = 0.0f;
    for (int k = lane; k < cols; k += 64) amax = fmaxf(amax, fabsf(val(k)));
    amax = wave_max(amax);
    const float sc = amax > 0.0f ? amax / 448.0f : 1.0f;
    uint8_t* row = dst + gr * stride;
    for (int k = lane; k < cols; k += 64) row[perm_stored8(k, cols)] = f32_to_e4m3(val(k) / sc);
    if (lane < 4) ((uint32_t*)(row + cols))[lane] = lane == 0 ? f2bits(sc) : 0u;
  }
}

}  // namespace mk
