// Calibration and probe kernels for gfx950, built as their own library (libetxmk_calib.so), outside the decode ABI:
//  - the cost of one grid barrier of the persistent decode kernels: the same grid_arrive / grid_wait (hierarchical
//    arrival over 8 group counters, 8 release flags, bounded wait) that etxmk_fused runs between phases, here back
//    to back with no work between them, one 512-thread workgroup per CU, cooperative launch;
//  - the HBM read bandwidth of the decode kernels' streaming pattern: non-temporal 16-byte loads, 1 KiB per wave
//    per load (64 lanes x 16 bytes), INF such loads issued before any is used, at 1, 2, 4, 8 and 16 in flight;
//  - the matrix-core probe: chained v_mfma_f32_16x16x32_bf16 on register contents the caller lays out, one wave
//    per case, so that the instruction's accumulation can be compared with a CPU statement of it.
// The stream kernel sums every 32-bit word it reads into a per-thread sink (mod 2^32) so that the loads cannot be
// dropped and the caller can check that every byte was read exactly once.
#include "mk_device.h"

namespace mk {
namespace {

struct CalibSmem {
  int32_t phase;
  int32_t abort;
};

__global__ __launch_bounds__(NT) void calib_barrier(Params p, int iters) {
  __shared__ CalibSmem s;
  if (threadIdx.x == 0) s.abort = 0;
  __syncthreads();
  int k = 0;
  for (int i = 0; i < iters; ++i) {
    grid_arrive(p, k, s);
    if (!grid_wait(p, k, s)) return;
  }
}

// wave w reads 1 KiB chunks w + W * (INF * t + j), j = 0 .. INF - 1, issuing the INF loads of a round together
template <int INF>
__global__ __launch_bounds__(NT) void calib_stream(const u32x4* src, size_t nchunk, uint32_t* sink) {
  const size_t W = (size_t)gridDim.x * NWAVE;
  const size_t w = (size_t)blockIdx.x * NWAVE + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  uint32_t acc = 0;
  for (size_t c = w; c < nchunk; c += W * INF) {
    u32x4 v[INF];
#pragma unroll
    for (int j = 0; j < INF; ++j) {
      const size_t cj = c + (size_t)j * W;
      v[j] = cj < nchunk ? ld_nt16(src + cj * 64 + lane) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < INF; ++j) acc += v[j].x + v[j].y + v[j].z + v[j].w;
  }
  sink[(size_t)blockIdx.x * NT + threadIdx.x] = acc;
}

// the matrix-core tiles' load pattern: wave w reads tiles of 16 consecutive rows (row_bytes apart), a tile's rows
// in blocks of 1024 bytes; one block is 16 loads per lane, lane (r = l % 16, q = l / 16) taking row r's bytes
// 16 q + 64 i of the block, i < 16 (64 bytes of every row per load, the other 64 of each 128-byte line in the next);
// INF blocks in flight
template <int INF>
__global__ __launch_bounds__(NT) void calib_stream_tiles(const uint8_t* src, int ntile, int nblk, int row_bytes,
                                                         uint32_t* sink) {
  const int W = gridDim.x * NWAVE, w = blockIdx.x * NWAVE + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
  const int nitem = (w < ntile ? (ntile - 1 - w) / W + 1 : 0) * nblk;
  uint32_t acc = 0;
  for (int it0 = 0; it0 < nitem; it0 += INF) {
    u32x4 v[INF][16];
#pragma unroll
    for (int j = 0; j < INF; ++j) {
      const int it = it0 + j;
      const bool ok = it < nitem;
      const int t = w + (it / nblk) * W, blk = it % nblk;
      const uint8_t* base = src + ((size_t)16 * t + r) * row_bytes + 1024 * blk + 16 * q;
#pragma unroll
      for (int i = 0; i < 16; ++i) v[j][i] = ok ? *(const u32x4*)(base + 64 * i) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < INF; ++j)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc += v[j][i].x + v[j][i].y + v[j][i].z + v[j][i].w;
  }
  sink[(size_t)blockIdx.x * NT + threadIdx.x] = acc;
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// lane i of case blockIdx.x: a, b hold nsteps blocks of 8 bf16 per lane, c and d 4 floats per lane
__global__ __launch_bounds__(64) void calib_mfma_bf16(const u32x4* a, const u32x4* b, const f32x4* c, f32x4* d,
                                                      int nsteps) {
  const size_t i = (size_t)blockIdx.x * 64 + threadIdx.x;
  f32x4 acc = c[i];
  for (int s = 0; s < nsteps; ++s) {
    const bf16x8 av = __builtin_bit_cast(bf16x8, a[i * nsteps + s]);
    const bf16x8 bv = __builtin_bit_cast(bf16x8, b[i * nsteps + s]);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
  }
  d[i] = acc;
}

int co_resident(const void* fn) {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, NT, 0) != hipSuccess) return -1;
  return cus * per_cu;
}

}  // namespace
}  // namespace mk

extern "C" {

// iters grid barriers in one cooperative launch of nwg workgroups.  bar: 17 * 64 uint32, zero on entry (the
// barrier's generations start at 1); abort_word: one int32, zero on entry, nonzero afterwards if a wait gave up
// (2: its 2 s limit).  Returns 0, or the HIP error code (hipErrorInvalidValue for a grid that is not co-resident).
int etxmk_calib_barrier(uint32_t* bar, int32_t* abort_word, int nwg, int iters, void* stream) {
  using namespace mk;
  if (!bar || !abort_word || nwg < 8 || iters < 0) return (int)hipErrorInvalidValue;
  const int most = co_resident((const void*)calib_barrier);
  if (most < 0) return (int)hipErrorInvalidDevice;
  if (nwg > most) return (int)hipErrorInvalidValue;
  Params p{};
  p.bar = bar;
  p.bar_base = 0;
  p.abort_word = abort_word;
  p.host_stop = nullptr;
  p.trace = nullptr;
  p.nwg = nwg;
  p.spin_ticks = 200000000ull;          // 2 s at the 100 MHz real-time clock
  p.poll_mask = 255;
  void* args[] = {&p, &iters};
  const hipError_t e = hipLaunchCooperativeKernel((const void*)calib_barrier, dim3(nwg), dim3(NT), args, 0,
                                                  (hipStream_t)stream);
  return e == hipSuccess ? (int)hipGetLastError() : (int)e;
}

// one streaming read of bytes (a multiple of 1024) at src with inflight (1, 2, 4, 8 or 16) 1 KiB loads per wave
// in flight, nwg workgroups of 512 threads; sink: nwg * 512 uint32, each thread's sum of the words it read.
int etxmk_calib_stream(const void* src, size_t bytes, int inflight, int nwg, uint32_t* sink, void* stream) {
  using namespace mk;
  if (!src || !sink || nwg < 1 || bytes % 1024 != 0 || ((uintptr_t)src & 15) != 0) return (int)hipErrorInvalidValue;
  const size_t nchunk = bytes / 1024;
  const u32x4* s = (const u32x4*)src;
  hipStream_t st = (hipStream_t)stream;
  switch (inflight) {
    case 1: hipLaunchKernelGGL(calib_stream<1>, dim3(nwg), dim3(NT), 0, st, s, nchunk, sink); break;
    case 2: hipLaunchKernelGGL(calib_stream<2>, dim3(nwg), dim3(NT), 0, st, s, nchunk, sink); break;
    case 4: hipLaunchKernelGGL(calib_stream<4>, dim3(nwg), dim3(NT), 0, st, s, nchunk, sink); break;
    case 8: hipLaunchKernelGGL(calib_stream<8>, dim3(nwg), dim3(NT), 0, st, s, nchunk, sink); break;
    case 16: hipLaunchKernelGGL(calib_stream<16>, dim3(nwg), dim3(NT), 0, st, s, nchunk, sink); break;
    default: return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}

// one read of ntile tiles of 16 rows (row_bytes apart, nblk blocks of 1024 bytes each) with the matrix-core tiles'
// load pattern, inflight (1 or 2) blocks of 16 KB per wave in flight, nwg workgroups of 512 threads; sink as above
int etxmk_calib_stream_tiles(const void* src, int ntile, int nblk, int row_bytes, int inflight, int nwg, uint32_t* sink,
                             void* stream) {
  using namespace mk;
  if (!src || !sink || nwg < 1 || ntile < 1 || nblk < 1 || row_bytes < 1024 * nblk || row_bytes % 16 ||
      ((uintptr_t)src & 15) != 0)
    return (int)hipErrorInvalidValue;
  const uint8_t* s = (const uint8_t*)src;
  hipStream_t st = (hipStream_t)stream;
  switch (inflight) {
    case 1: hipLaunchKernelGGL(calib_stream_tiles<1>, dim3(nwg), dim3(NT), 0, st, s, ntile, nblk, row_bytes, sink); break;
    case 2: hipLaunchKernelGGL(calib_stream_tiles<2>, dim3(nwg), dim3(NT), 0, st, s, ntile, nblk, row_bytes, sink); break;
    default: return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}

// ncase waves, each nsteps chained v_mfma_f32_16x16x32_bf16 (D = C + A B, K = 32 per step) on per-lane register
// contents: a, b [ncase][64][nsteps][8] bf16 bits, c, d [ncase][64][4] fp32 (16-byte aligned).
int etxmk_calib_mfma_bf16(const uint16_t* a, const uint16_t* b, const float* c, float* d, int ncase, int nsteps,
                          void* stream) {
  using namespace mk;
  if (!a || !b || !c || !d || ncase < 1 || nsteps < 1 || nsteps > 4096) return (int)hipErrorInvalidValue;
  if ((((uintptr_t)a | (uintptr_t)b | (uintptr_t)c | (uintptr_t)d) & 15) != 0) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(calib_mfma_bf16, dim3(ncase), dim3(64), 0, (hipStream_t)stream, (const u32x4*)a, (const u32x4*)b,
                     (const f32x4*)c, (f32x4*)d, nsteps);
  return (int)hipGetLastError();
}

}  // extern "C"
