// Device pool build: the chunk operators of a document cache (fp16 slot rows per chunk) become
// fp16 pages and fp32 summary keys in one kernel (the math of Library.__init__ + _summaries,
// xenc/library.py:47-74):
//   optional centering:  row <- (row - mu) / (|row - mu| + 1e-6)   on valid rows
//   page c               = the chunk's rows, zero-padded to slots_per_page x d_pad
//   S[c]                 = m / (|m| + 1e-6),  m = sum of the valid rows / max(n_c, 1)
// One workgroup (8 waves) per chunk; wave w takes rows w, w + 8, ...; a lane owns 8 consecutive
// dims of each 512-dim block.  Row norms are wave reductions; the per-wave column sums merge in a
// fixed halving tree through LDS (deterministic), and wave 0 normalises and writes S.
#include <algorithm>

#include "xenc_common.h"

namespace xenc {
namespace {

constexpr int kPoolWaves = 8;
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

// Rows per wave per step, their loads issued together: more for narrow rows, fewer where the
// registers of wide rows would spill.
template <int CB>
constexpr int pool_rows() { return CB <= 2 ? 4 : (CB <= 6 ? 2 : 1); }

template <int CB>
__global__ __launch_bounds__(kPoolWaves * kWave) void build_pages_kernel(
    const _Float16* __restrict__ rows, const long long* __restrict__ row_off, int d,
    const float* __restrict__ mu, int N, int d_pad, _Float16* __restrict__ pages,
    long long page_stride, float* __restrict__ S, long long lds_s, int* __restrict__ nvalid) {
  extern __shared__ float red[];   // [kPoolWaves / 2][d_pad]
  const int c = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const long long r0 = row_off[c];
  const int n = (int)min(row_off[c + 1] - r0, (long long)N);
  float mv[CB][8], sum[CB][8];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int d0 = (cb * kWave + lane) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      mv[cb][e] = (mu && d0 + e < d) ? mu[d0 + e] : 0.f;
      sum[cb][e] = 0.f;
    }
  }
  _Float16* page = pages + (long long)c * page_stride;
  constexpr int kRows = pool_rows<CB>();
  // kRows rows per wave per step (t, t + kPoolWaves, ...): all their loads are issued before any
  // is used, multiplying the bytes in flight.  Rows are read once and pages written once, so both
  // go around the caches (nontemporal).
  for (int t0 = wv; t0 < N; t0 += kRows * kPoolWaves) {
    half8_t h[kRows][CB];
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
      const int t = t0 + u * kPoolWaves;
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int d0 = (cb * kWave + lane) * 8;
        h[u][cb] = half8_t{};
        if (t < n && d0 < d)
          h[u][cb] = __builtin_nontemporal_load(reinterpret_cast<const half8_t*>(rows + (r0 + t) * d + d0));
      }
    }
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
      const int t = t0 + u * kPoolWaves;
      if (t >= N) break;   // wave-uniform
      float x[CB][8];
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int d0 = (cb * kWave + lane) * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          x[cb][e] = (t < n && d0 + e < d) ? (float)h[u][cb][e] - mv[cb][e] : 0.f;
      }
      if (mu) {   // centre and renormalise the valid row
        float ss = 0.f;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
          for (int e = 0; e < 8; ++e) ss = fmaf(x[cb][e], x[cb][e], ss);
        const float inv = 1.f / (sqrtf(wave_sum(ss)) + 1e-6f);
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
          for (int e = 0; e < 8; ++e) x[cb][e] *= inv;
      }
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int d0 = (cb * kWave + lane) * 8;
        if (d0 < d_pad) {
          half8_t o;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            o[e] = (_Float16)x[cb][e];
            sum[cb][e] += x[cb][e];
          }
          __builtin_nontemporal_store(o, reinterpret_cast<half8_t*>(page + (long long)t * d_pad + d0));
        }
      }
    }
  }
  // Column sums of the 8 waves: halving tree, rounds h = 4, 2, 1.
  for (int h = kPoolWaves / 2; h >= 1; h /= 2) {
    if (wv >= h && wv < 2 * h) {
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int d0 = (cb * kWave + lane) * 8;
        if (d0 < d_pad)
#pragma unroll
          for (int e = 0; e < 8; ++e) red[(wv - h) * d_pad + d0 + e] = sum[cb][e];
      }
    }
    __syncthreads();
    if (wv < h) {
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int d0 = (cb * kWave + lane) * 8;
        if (d0 < d_pad)
#pragma unroll
          for (int e = 0; e < 8; ++e) sum[cb][e] += red[wv * d_pad + d0 + e];
      }
    }
    __syncthreads();
  }
  if (wv == 0) {
    const float cnt = (float)max(n, 1);
    float ss = 0.f;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sum[cb][e] /= cnt;
        ss = fmaf(sum[cb][e], sum[cb][e], ss);
      }
    const float inv = 1.f / (sqrtf(wave_sum(ss)) + 1e-6f);
    float* srow = S + (long long)c * lds_s;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int d0 = (cb * kWave + lane) * 8;
      if (d0 < d_pad)
#pragma unroll
        for (int e = 0; e < 8; ++e) srow[d0 + e] = sum[cb][e] * inv;
    }
    if (lane == 0) nvalid[c] = n;
  }
}

}  // namespace
}  // namespace xenc

using namespace xenc;

extern "C" int xenc_build_pages(const void* rows, const long long* row_off, int C, int d,
                                const float* mu, int slots_per_page, int d_pad, void* pages,
                                long long page_stride, float* S, long long lds, int* nvalid,
                                void* stream) {
  if (C < 0 || d <= 0 || d % 8 != 0 || d_pad < d || d_pad % 8 != 0 || d_pad > 8 * 512) return XENC_EINVAL;
  if (slots_per_page <= 0 || page_stride < (long long)slots_per_page * d_pad || lds < d_pad)
    return XENC_EINVAL;
  if (C == 0) return XENC_OK;
  if (!rows || !row_off || !pages || !S || !nvalid) return XENC_ENULL;
  if (!aligned16(rows) || !aligned16(pages) || page_stride % 8 != 0) return XENC_EALIGN;
  const size_t lds_bytes = (size_t)(kPoolWaves / 2) * d_pad * sizeof(float);
  if (lds_bytes > 64 * 1024) return XENC_EINVAL;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int cb = (d_pad + 511) / 512;
  const _Float16* r = static_cast<const _Float16*>(rows);
  _Float16* p = static_cast<_Float16*>(pages);
  switch (cb) {
#define XENC_POOL(N)                                                                              \
  case N:                                                                                         \
    hipLaunchKernelGGL(build_pages_kernel<N>, dim3(C), dim3(kPoolWaves * kWave), lds_bytes, st, r, \
                       row_off, d, mu, slots_per_page, d_pad, p, page_stride, S, lds, nvalid);    \
    break;
    XENC_POOL(1) XENC_POOL(2) XENC_POOL(3) XENC_POOL(4) XENC_POOL(5) XENC_POOL(6) XENC_POOL(7)
    XENC_POOL(8)
#undef XENC_POOL
    default:
      return XENC_EINVAL;
  }
  return check_launch();
}
