// Write-back of the read through the interface's B (the write of the epilogue,
// xenc/injector.py:71-74 and 266-267), for the decode path's few query rows:
//   out[m, o] = row_scale[m] * (sum_k W_g[o, k] r[m, k] + b_g[o]),   g = row_group[m]
// row_scale carries gain_scale * exp(log_gain) * gate per row.  W_g is the fp32 [d_out, d]
// weight of library (depth) g.  This is an HBM-bound skinny GEMM: every W row a used library
// needs is streamed once (rows of unused libraries are not read), while the query rows stay in
// the caches.
//
// One workgroup (4 waves) per (tile of output rows, library g, batch of up to 8 of g's rows);
// wave w owns kWbOut output rows.  Lanes run along k (4 consecutive k each, so a W row is read
// as coalesced 1 KiB loads), and a wave keeps kWbOut outputs x kWbRows query rows of partial
// sums.  The rows of library g are listed (ascending) by a ballot compaction.  A reduce-scatter
// across the lanes finishes the dot products; each (row, output) is written by one lane, in a
// fixed summation order (deterministic).
#include <algorithm>

#include "xenc_common.h"

namespace xenc {
namespace {

#ifndef XENC_WB_OUT
#define XENC_WB_OUT 8
#endif
#ifndef XENC_WB_ROWS
#define XENC_WB_ROWS 8
#endif
#ifndef XENC_WB_WAVES
#define XENC_WB_WAVES 4
#endif
constexpr int kWbWaves = XENC_WB_WAVES;
constexpr int kWbOut = XENC_WB_OUT;    // output rows per wave
constexpr int kWbRows = XENC_WB_ROWS;  // query rows per batch
constexpr int kWbMaxRows = 4096;    // query rows per call
constexpr int kWbMaxGroups = 1024;  // libraries per call
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float dot4(const f32x4& a, const f32x4& b, float acc) {
  acc = fmaf(a[0], b[0], acc);
  acc = fmaf(a[1], b[1], acc);
  acc = fmaf(a[2], b[2], acc);
  return fmaf(a[3], b[3], acc);
}

// Work item = (output tile, library g, batch b of g's rows): the items of one tile and library
// are adjacent in the XCD-major launch order, so the batches of a library with more than
// kWbRows rows read the same W rows at the same time on one XCD (L2 hits after the first).
// An item index past the last (library, batch) pair exits at once.
__global__ __launch_bounds__(kWbWaves * kWave) void write_back_kernel(
    const float* __restrict__ r, long long ldr, int M, int d, const int* __restrict__ row_group,
    int G, const float* __restrict__ W, long long wgs, long long ldw, int d_out,
    const float* __restrict__ bias, long long bgs, const float* __restrict__ row_scale,
    float* __restrict__ out, long long ldo, int n_pairs) {
  __shared__ int list[kWbMaxRows];
  __shared__ int hist[kWbMaxGroups];
  __shared__ int wcount[kWbWaves];
  __shared__ int pair_g, pair_b;
  constexpr int kTile = kWbWaves * kWbOut;
  const int item = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = item / n_pairs;
  const int p = item % n_pairs;
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  auto group_of = [&](int m) { return min(max(row_group ? row_group[m] : 0, 0), G - 1); };

  // (library, batch) of pair p: libraries in order, ceil(n_g / kWbRows) batches each.  The row
  // counts come from one LDS histogram pass (integer counts: order-independent).
  for (int g = threadIdx.x; g < G; g += kWbWaves * kWave) hist[g] = 0;
  __syncthreads();
  for (int m = threadIdx.x; m < M; m += kWbWaves * kWave) atomicAdd(&hist[group_of(m)], 1);
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc_pairs = 0, gg = -1, bb = 0;
    for (int g = 0; g < G; ++g) {
      const int nb = (hist[g] + kWbRows - 1) / kWbRows;
      if (p < acc_pairs + nb) {
        gg = g;
        bb = p - acc_pairs;
        break;
      }
      acc_pairs += nb;
    }
    pair_g = gg;
    pair_b = bb;
  }
  __syncthreads();
  const int g = pair_g, batch = pair_b;
  if (g < 0) return;

  // Rows of library g in ascending order.
  int n = 0;
  for (int base = 0; base < M; base += kWbWaves * kWave) {
    const int m = base + threadIdx.x;
    const bool f = m < M && group_of(m) == g;
    const unsigned long long bal = __ballot(f);
    if (lane == 0) wcount[wv] = __popcll(bal);
    __syncthreads();
    int off = n, tot = 0;
#pragma unroll
    for (int w = 0; w < kWbWaves; ++w) {
      off += w < wv ? wcount[w] : 0;
      tot += wcount[w];
    }
    if (f) list[off + __popcll(bal & ((1ull << lane) - 1ull))] = m;
    n += tot;
    __syncthreads();
  }

  const int o0 = tile * kTile + wv * kWbOut;
  const float* Wg = W + (long long)g * wgs;
  const bool shared_w = n > kWbRows;  // sibling batches read these W rows too: keep them cached
  const int b0 = batch * kWbRows;
  const float* rp[kWbRows];
#pragma unroll
  for (int j = 0; j < kWbRows; ++j) rp[j] = b0 + j < n ? r + (long long)list[b0 + j] * ldr : nullptr;
  float acc[kWbOut * kWbRows];
#pragma unroll
  for (int i = 0; i < kWbOut * kWbRows; ++i) acc[i] = 0.f;
#ifdef XENC_WB_UNROLL
#pragma unroll XENC_WB_UNROLL
#endif
  for (int k = lane * 4; k < d; k += kWave * 4) {
    f32x4 wr[kWbOut], qr[kWbRows];
#pragma unroll
    for (int i = 0; i < kWbOut; ++i) {
      const int o = o0 + i;
      wr[i] = f32x4{};
      if (o < d_out) {
        const f32x4* pw = reinterpret_cast<const f32x4*>(Wg + (long long)o * ldw + k);
        wr[i] = shared_w ? *pw : __builtin_nontemporal_load(pw);
      }
    }
#pragma unroll
    for (int j = 0; j < kWbRows; ++j)
      qr[j] = rp[j] ? *reinterpret_cast<const f32x4*>(rp[j] + k) : f32x4{};
#pragma unroll
    for (int i = 0; i < kWbOut; ++i)
#pragma unroll
      for (int j = 0; j < kWbRows; ++j) acc[i * kWbRows + j] = dot4(wr[i], qr[j], acc[i * kWbRows + j]);
  }
  // Reduce-scatter of the kWbOut * kWbRows sums: lane l ends with the full sum of value
  // l / kRep (kRep lanes hold each value; the first of them writes it).
  constexpr int kVals = kWbOut * kWbRows;
  constexpr int kRep = kWave / kVals;
  wave_reduce_scatter<kVals>(acc, lane);
  const int v = lane / kRep;
  const int i = v / kWbRows, j = v % kWbRows;
  const int o = o0 + i;
  if (lane % kRep == 0 && o < d_out && b0 + j < n) {
    const int m = list[b0 + j];
    float y = acc[0] + (bias ? bias[(long long)g * bgs + o] : 0.f);
    if (row_scale) y *= row_scale[m];
    out[(long long)m * ldo + o] = y;
  }
}

}  // namespace
}  // namespace xenc

using namespace xenc;

extern "C" int xenc_write_back(const float* r, long long ldr, int M, int d, const int* row_group,
                               int G, const float* W, long long w_group_stride, long long ldw,
                               int d_out, const float* bias, long long bias_group_stride,
                               const float* row_scale, float* out, long long ldo, void* stream) {
  if (M < 0 || M > kWbMaxRows || d <= 0 || d % 4 != 0 || G <= 0 || G > kWbMaxGroups || d_out <= 0)
    return XENC_EINVAL;
  if (ldr < d || ldr % 4 != 0 || ldw < d || ldw % 4 != 0 || ldo < d_out) return XENC_EINVAL;
  if (G > 1 && w_group_stride < (long long)d_out * ldw) return XENC_EINVAL;
  if (bias && G > 1 && bias_group_stride != 0 && bias_group_stride < d_out) return XENC_EINVAL;
  if (M == 0) return XENC_OK;
  if (!r || !W || !out) return XENC_ENULL;
  if (!aligned16(r) || !aligned16(W) || (G > 1 && w_group_stride % 4 != 0)) return XENC_EALIGN;
  const long long tiles = (d_out + kWbWaves * kWbOut - 1) / (kWbWaves * kWbOut);
  // (library, batch) pairs: sum over libraries of ceil(n_g / kWbRows) <= min(G, M) + M / kWbRows.
  const long long n_pairs = std::min<long long>(G, M) + M / kWbRows;
  if (n_pairs * tiles > 0x7fffffffLL) return XENC_EINVAL;
  hipLaunchKernelGGL(write_back_kernel, dim3((unsigned)(n_pairs * tiles)), dim3(kWbWaves * kWave), 0,
                     reinterpret_cast<hipStream_t>(stream), r, ldr, M, d, row_group, G, W,
                     w_group_stride, ldw, d_out, bias, bias_group_stride, row_scale, out, ldo,
                     (int)n_pairs);
  return check_launch();
}
