// Calibration kernels for the roofline denominators, measured on the device the reads run on
// (the vendor peaks assume clocks this part does not hold under sustained load):
//
//   mfma_rate_kernel    every wave issues rounds of 16 independent v_mfma_f32_32x32x16_f16 on
//                       register operands loaded once from random fp16 data (two operand sets
//                       alternated, so the inputs keep toggling); nothing but the final sums
//                       touches memory.  The fp16 MFMA rate the chip sustains.
//   stream_read_kernel  16-byte nontemporal loads, each workgroup over a contiguous range with
//                       eight loads in flight per lane, one value per lane written at the end:
//                       the HBM read rate the decode kernels stream at.
#include "xenc_common.h"

namespace xenc {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void mfma_rate_kernel(const half8_t* __restrict__ src, int n_src,
                                                        int rounds, float* __restrict__ out) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  const half8_t a0 = src[(4 * t) % n_src], b0 = src[(4 * t + 1) % n_src];
  const half8_t a1 = src[(4 * t + 2) % n_src], b1 = src[(4 * t + 3) % n_src];
  f32x16 acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = (f32x16){};
  for (int it = 0; it < rounds; ++it) {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16((j & 1) ? a1 : a0, (j & 2) ? b1 : b0, acc[j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[j][r];
  out[t] = s;
}

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ src, long long n16,
                                                          long long per_block, float* __restrict__ out) {
  // Workgroup b reads its contiguous range [b * per_block, (b + 1) * per_block) of 16-byte
  // vectors, eight loads in flight per lane.
  const long long beg = blockIdx.x * per_block;
  const long long end = min(n16, beg + per_block);
  unsigned acc = 0;
  long long i = beg + threadIdx.x;
  constexpr int U = 8;
  for (; i + (U - 1) * 256 < end; i += U * 256) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(src + i + u * 256);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];   // all 16 bytes live
  }
  for (; i < end; i += 256) {
    const u32x4 t = __builtin_nontemporal_load(src + i);
    acc ^= t[0] ^ t[1] ^ t[2] ^ t[3];
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = (float)acc;
}

}  // namespace
}  // namespace xenc

using namespace xenc;

extern "C" int xenc_calibrate_mfma(const void* src, int n_src, int waves_per_cu, int cus, int rounds,
                                   float* out, void* stream) {
  if (n_src < 4 || waves_per_cu < 4 || waves_per_cu % 4 != 0 || cus <= 0 || rounds <= 0) return XENC_EINVAL;
  if (!src || !out) return XENC_ENULL;
  if (!aligned16(src)) return XENC_EALIGN;
  hipLaunchKernelGGL(mfma_rate_kernel, dim3(cus * waves_per_cu / 4), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const half8_t*>(src), n_src, rounds,
                     out);
  return check_launch();
}

extern "C" int xenc_calibrate_stream(const void* src, long long bytes, int blocks, float* out, void* stream) {
  if (bytes < 16 || bytes % 16 != 0 || blocks <= 0) return XENC_EINVAL;
  if (!src || !out) return XENC_ENULL;
  if (!aligned16(src)) return XENC_EALIGN;
  const long long n16 = bytes / 16;
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), n16, (n16 + blocks - 1) / blocks, out);
  return check_launch();
}
