// Device numerics of the decode step (gfx950).  Every function here is the device side of a rule the
// CPU oracle states independently; the pair is compared bit for bit by the GPU parity tests.
//
//  * bf16 round-to-nearest-even at the points examples/llm/ref_numpy.py:26-32 (bfr) rounds.
//  * exp: Cody-Waite reduction by ln2 and a degree-7 Taylor polynomial, IEEE single operations only.
//  * seeded weights: splitmix64 counter stream (Steele, Lea, Flood 2014) and Box-Muller with
//    polynomial log / sin / cos, again only +, *, /, sqrt and fma, so host and device agree exactly.
//  * dot order: lane l of a wave64 accumulates elements k = l (mod 64) in ascending k with fma;
//    lanes are combined by wave_sum() below.
//
// The library is compiled with -ffp-contract=off: every fma below is explicit.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mk {

__device__ __forceinline__ float bits2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2bits(float f) { return __float_as_uint(f); }

// round to bf16 (RNE), kept in fp32
__device__ __forceinline__ float bfr(float x) {
  uint32_t u = f2bits(x);
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  return bits2f(u);
}
__device__ __forceinline__ uint16_t f2bf(float x) {
  const uint32_t u = f2bits(x);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float bf2f(uint16_t b) { return bits2f((uint32_t)b << 16); }
__device__ __forceinline__ float bf_lo(uint32_t w) { return bits2f(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return bits2f(w & 0xFFFF0000u); }

__device__ __forceinline__ float expf_mk(float x) {
  if (!(x > -87.0f)) return (x != x) ? x : 0.0f;
  if (x > 88.72283f) return __builtin_huge_valf();
  const float n = floorf(__builtin_fmaf(x, 1.44269504f, 0.5f));
  float r = __builtin_fmaf(n, -0.693359375f, x);
  r = __builtin_fmaf(n, 2.12194440e-4f, r);
  float p = 1.98412698e-4f;
  p = __builtin_fmaf(p, r, 1.38888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int ni = (int)n, h = ni / 2, g = ni - h;
  const float s1 = bits2f((uint32_t)(h + 127) << 23), s2 = bits2f((uint32_t)(g + 127) << 23);
  return (p * s1) * s2;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf_mk(-g)); }

// ---------------------------------------------------------------- seeded generator
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__host__ __device__ __forceinline__ uint64_t stream_key(uint64_t seed, uint64_t stream) { return mix64(mix64(seed) ^ stream); }
__host__ __device__ __forceinline__ uint64_t stream_bits(uint64_t key, uint64_t i) {
  return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull);
}

__device__ __forceinline__ float log_unit(float u) {          // ln u, u in (0, 1]
  const uint32_t b = f2bits(u);
  int e = (int)((b >> 23) & 0xFF) - 127;
  float m = bits2f((b & 0x007FFFFFu) | 0x3F800000u);
  if (m > 1.41421356f) { m = m * 0.5f; e += 1; }
  const float s = (m - 1.0f) / (m + 1.0f), s2 = s * s;
  float p = 7.69230769e-2f;
  p = __builtin_fmaf(p, s2, 9.09090909e-2f);
  p = __builtin_fmaf(p, s2, 1.11111111e-1f);
  p = __builtin_fmaf(p, s2, 1.42857143e-1f);
  p = __builtin_fmaf(p, s2, 2.00000000e-1f);
  p = __builtin_fmaf(p, s2, 3.33333333e-1f);
  p = __builtin_fmaf(p, s2, 1.0f);
  const float lnm = 2.0f * s * p;
  const float fe = (float)e;
  return __builtin_fmaf(fe, 0.693145752f, __builtin_fmaf(fe, 1.42860677e-6f, lnm));
}

__device__ __forceinline__ void sincos_quadrant(float phi, float& s, float& c) {   // phi in [0, pi/2)
  const float x2 = phi * phi;
  float ps = 1.60590438e-10f;
  ps = __builtin_fmaf(ps, x2, -2.50521084e-8f);
  ps = __builtin_fmaf(ps, x2, 2.75573192e-6f);
  ps = __builtin_fmaf(ps, x2, -1.98412698e-4f);
  ps = __builtin_fmaf(ps, x2, 8.33333333e-3f);
  ps = __builtin_fmaf(ps, x2, -1.66666667e-1f);
  ps = __builtin_fmaf(ps, x2, 1.0f);
  s = phi * ps;
  float pc = -1.14707456e-11f;
  pc = __builtin_fmaf(pc, x2, 2.08767570e-9f);
  pc = __builtin_fmaf(pc, x2, -2.75573192e-7f);
  pc = __builtin_fmaf(pc, x2, 2.48015873e-5f);
  pc = __builtin_fmaf(pc, x2, -1.38888889e-3f);
  pc = __builtin_fmaf(pc, x2, 4.16666667e-2f);
  pc = __builtin_fmaf(pc, x2, -0.5f);
  pc = __builtin_fmaf(pc, x2, 1.0f);
  c = pc;
}

// standard normal number i of the stream with key `key` (Box-Muller on pair i/2)
__device__ __forceinline__ float normal_at(uint64_t key, uint64_t i) {
  const uint64_t bits = stream_bits(key, i >> 1);
  const uint32_t a = (uint32_t)(bits >> 40), b = (uint32_t)((bits >> 16) & 0xFFFFFFu);
  const float u1 = (float)(a + 1u) * 5.96046448e-8f;
  const float r = __builtin_sqrtf(-2.0f * log_unit(u1));
  const uint32_t q = b >> 22;
  const float phi = (float)(b & 0x3FFFFFu) * 2.38418579e-7f * 1.57079637f;
  float s, c;
  sincos_quadrant(phi, s, c);
  const float cs = q == 0 ? c : q == 1 ? -s : q == 2 ? -c : s;
  const float sn = q == 0 ? s : q == 1 ? c : q == 2 ? -s : -c;
  return r * ((i & 1) ? sn : cs);
}

// ---------------------------------------------------------------- lane-permuted rows
// A row of K bf16 weights is stored in blocks of 512 (the last block may hold 64*m < 512); inside a block
// lane l's m = size/64 consecutive stored elements are the logical elements l, l+64, ..., l+64(m-1).  One
// 16-byte load then gives a lane exactly the elements its accumulator owns in the dot order above.
__host__ __device__ __forceinline__ int perm_logical(int p, int K) {   // stored position -> logical element
  const int base = p & ~511;
  const int S = (K - base) < 512 ? (K - base) : 512;
  const int m = S >> 6;
  const int q = p - base;
  return base + q / m + 64 * (q % m);
}
__host__ __device__ __forceinline__ int perm_stored(int k, int K) {    // logical element -> stored position
  const int base = k & ~511;
  const int S = (K - base) < 512 ? (K - base) : 512;
  const int m = S >> 6;
  const int q = k - base;
  return base + (q & 63) * m + (q >> 6);
}
// logical element k of an fp8 row -> its stored byte (blocks of 1024; lane l holds l, l+64, ...)
__host__ __device__ __forceinline__ int perm_stored8(int k, int K) {
  const int base = k & ~1023;
  const int S = (K - base) < 1024 ? (K - base) : 1024;
  const int m = S >> 6;
  const int q = k - base;
  return base + (q & 63) * m + (q >> 6);
}

// Lane reduction of a wave64 in the fixed order the CPU oracle restates: partner l^1, then l^2 (DPP quad
// permutes), then the mirror inside 8 lanes and inside 16 lanes (DPP row_half_mirror, row_mirror); each 16-lane row
// then holds its sum in every lane, and the four rows are combined as (row0 + row1) + (row2 + row3).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum(float v) {
  v = v + dpp_mov<0xB1>(v);     // quad_perm [1,0,3,2]
  v = v + dpp_mov<0x4E>(v);     // quad_perm [2,3,0,1]
  v = v + dpp_mov<0x141>(v);    // row_half_mirror
  v = v + dpp_mov<0x140>(v);    // row_mirror
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}
// max is exact in any order: the same DPP row steps, then the four rows through readlane (no LDS round trips)
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  v = fmaxf(v, dpp_mov<0x140>(v));
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// ---------------------------------------------------------------- global-memory access
// Pointers that reach the kernels through structures are generic; dereferencing them directly makes flat
// instructions, which also count against the LDS counter (so every LDS wait would wait for the weight stream
// too).  Every device-memory access therefore goes through an address-space-1 (global) pointer.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#define MK_G __attribute__((address_space(1)))

__device__ __forceinline__ u32x4 ld_nt16(const void* p) { return __builtin_nontemporal_load((const MK_G u32x4*)p); }
__device__ __forceinline__ uint32_t ld_nt4(const void* p) { return __builtin_nontemporal_load((const MK_G uint32_t*)p); }
__device__ __forceinline__ u32x4 ld16(const void* p) { return *(const MK_G u32x4*)p; }
__device__ __forceinline__ uint32_t ld4(const void* p) { return *(const MK_G uint32_t*)p; }
__device__ __forceinline__ uint16_t ld_u16(const uint16_t* p) { return *(const MK_G uint16_t*)p; }
__device__ __forceinline__ float ld_f(const float* p) { return *(const MK_G float*)p; }
__device__ __forceinline__ int32_t ld_i(const int32_t* p) { return *(const MK_G int32_t*)p; }
__device__ __forceinline__ void st_u16(uint16_t* p, uint16_t v) { *(MK_G uint16_t*)p = v; }
__device__ __forceinline__ void st_f(float* p, float v) { *(MK_G float*)p = v; }
__device__ __forceinline__ void st_i(int32_t* p, int32_t v) { *(MK_G int32_t*)p = v; }

// agent-scope (cross-XCD coherent) element access for activations shared between workgroups
__device__ __forceinline__ float ld_ag(const float* p) {
  return __uint_as_float(__hip_atomic_load((const MK_G uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void st_ag(float* p, float v) {
  __hip_atomic_store((MK_G uint32_t*)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_ag64(const uint64_t* p) {
  return __hip_atomic_load((const MK_G uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_ag_i(const int32_t* p) {
  return __hip_atomic_load((const MK_G int32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_ag_i(int32_t* p, int32_t v) {
  __hip_atomic_store((MK_G int32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// system-scope load of a word the host writes (pinned, device-mapped host memory)
__device__ __forceinline__ int32_t ld_sys_i(const int32_t* p) {
  return __hip_atomic_load((const MK_G int32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint16_t ld_ag_u16(const uint16_t* p) {
  return __hip_atomic_load((const MK_G uint16_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_ag_u16(uint16_t* p, uint16_t v) {
  __hip_atomic_store((MK_G uint16_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_ag_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store((MK_G uint32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// cache-policy operand of global_load_lds for an agent-coherent (sc1) load, like the agent-scope loads above
constexpr int LDS_SC1 = 16;

}  // namespace mk
