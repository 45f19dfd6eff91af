// Slot top-k selection read (D8, xenc/topk_read.py): the reader's query at a selection layer
// picks the k library slots whose selection keys score highest, and the read then runs over
// those k slots only, with one softmax.
//
//   select_scores_kernel  s[b, i] = pool_h <q[b, h], K[i, h / G]>  (pool = max or mean over the
//                         query heads, GQA group G = n_q / n_kv), -inf on invalid slots
//                         (xenc/topk_read.py:205-226)
//   topk_rows_kernel      the k largest s[b, :] per row, in descending order, ties to the lower
//                         index (xenc/topk_read.py:237-240; torch.topk leaves ties unspecified)
//   gather_pages_kernel   the selected slot rows copied, in selection order, into a compact page
//                         per selection set, zero-padded; the existing decode and MFMA read
//                         kernels then read that one-chunk library with route weight 1, which is
//                         the read of the selected set (xenc/topk_read.py:383-414)
#include <algorithm>

#include "xenc_common.h"

namespace xenc {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------
// Scores: one wave per (slot, query row); lanes run over hd for each kv head.  A workgroup of
// 4 waves takes 4 consecutive slots for one query row.  The keys dominate the traffic
// (n_kv * hd * 4 bytes per slot per query row); query rows are few (the batch at one position).
__global__ __launch_bounds__(256) void select_scores_kernel(
    const float* __restrict__ q, int n_q, int n_kv, int hd, const float* __restrict__ keys, int S,
    const unsigned char* __restrict__ valid, int pool_mean, float* __restrict__ scores, long long ld_s) {
  const int b = blockIdx.y;
  const int lane = threadIdx.x & (kWave - 1);
  const int i = blockIdx.x * 4 + threadIdx.x / kWave;
  if (i >= S) return;  // wave-uniform
  const int G = n_q / n_kv;
  float best = -INFINITY, sum = 0.f;
  for (int h = 0; h < n_q; ++h) {
    const float* qh = q + ((long long)b * n_q + h) * hd;
    const float* kh = keys + ((long long)i * n_kv + h / G) * hd;
    float p = 0.f;
    for (int e = lane; e < hd; e += kWave) p = fmaf(qh[e], kh[e], p);
    p = wave_sum(p);
    best = fmaxf(best, p);
    sum += p;
  }
  if (lane == 0) {
    const bool ok = valid == nullptr || valid[i] != 0;
    scores[(long long)b * ld_s + i] = ok ? (pool_mean ? sum / (float)n_q : best) : -INFINITY;
  }
}

// ------------------------------------------------------------------------------------------
// Top-k per row by radix select on an order-preserving integer key of the fp32 score:
// key(x) = bits(x) | 0x80000000 for x >= 0, ~bits(x) for x < 0 (larger x -> larger key).
// Four 8-bit passes (most significant byte first) narrow the k-th largest key T; the winners
// are every key > T plus the first (lowest-index) keys == T up to k, gathered in index order by
// a workgroup scan; a bitonic sort of the winners by (key desc, index asc) gives the order.
constexpr int kTopkThreads = 1024;
constexpr int kTopkMax = 1024;

__device__ __forceinline__ unsigned int order_key(float x) {
  const unsigned int u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inclusive scan of one int per thread over the workgroup (16 waves): wave scan with shuffles,
// wave totals through LDS.  Returns the inclusive prefix; *total = the workgroup sum.
__device__ __forceinline__ int block_scan(int v, int* wsum, int* total) {
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int t = __shfl_up(v, o, kWave);
    if (lane >= o) v += t;
  }
  if (lane == kWave - 1) wsum[wv] = v;
  __syncthreads();
  int off = 0, tot = 0;
  for (int w = 0; w < kTopkThreads / kWave; ++w) {
    off += w < wv ? wsum[w] : 0;
    tot += wsum[w];
  }
  __syncthreads();
  *total = tot;
  return v + off;
}

__global__ __launch_bounds__(kTopkThreads) void topk_rows_kernel(
    const float* __restrict__ scores, long long ld_s, int S, int k, int* __restrict__ idx,
    float* __restrict__ vals, long long ld_o) {
  __shared__ int hist[256];
  __shared__ int wsum[kTopkThreads / kWave];
  __shared__ unsigned int sel_key[kTopkMax];
  __shared__ int sel_idx[kTopkMax];
  __shared__ unsigned int prefix_s, mask_s;
  __shared__ int need_s;
  const int b = blockIdx.x;
  const float* row = scores + (long long)b * ld_s;
  const int tid = threadIdx.x;

  // Radix select of the k-th largest key.
  unsigned int prefix = 0, mask = 0;
  int need = k;  // how many of the keys matching `prefix` (under `mask`) still belong to the top k
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    for (int i = tid; i < S; i += kTopkThreads) {
      const unsigned int key = order_key(row[i]);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255], 1);
    }
    __syncthreads();
    if (tid == 0) {
      int acc = 0, bin = 255;
      for (; bin > 0; --bin) {
        if (acc + hist[bin] >= need) break;
        acc += hist[bin];
      }
      need_s = need - acc;
      prefix_s = prefix | ((unsigned int)bin << shift);
      mask_s = mask | (255u << shift);
    }
    __syncthreads();
    prefix = prefix_s;
    mask = mask_s;
    need = need_s;
  }
  const unsigned int T = prefix;  // the k-th largest key; `need` of the keys == T are taken

  // Winners in index order: keys > T, and keys == T while fewer than `need` were taken.
  int base_gt = 0, base_eq = 0;
  for (int i0 = 0; i0 < S; i0 += kTopkThreads) {
    const int i = i0 + tid;
    unsigned int key = 0;
    int gt = 0, eq = 0;
    if (i < S) {
      key = order_key(row[i]);
      gt = key > T;
      eq = key == T;
    }
    int tot_gt, tot_eq;
    const int pgt = block_scan(gt, wsum, &tot_gt) - gt;
    const int peq = block_scan(eq, wsum, &tot_eq) - eq;
    const int n_gt_total_before = base_gt + pgt;
    const int n_eq_before = base_eq + peq;
    // Output slot: all keys > T come first in index order, then the first `need` keys == T.
    if (gt) {
      const int pos = n_gt_total_before;
      sel_key[pos] = key;
      sel_idx[pos] = i;
    } else if (eq && n_eq_before < need) {
      const int pos = (k - need) + n_eq_before;
      sel_key[pos] = key;
      sel_idx[pos] = i;
    }
    base_gt += tot_gt;
    base_eq += tot_eq;
  }
  __syncthreads();

  // Bitonic sort of the k winners (padded to a power of two) by (key desc, index asc).
  int P = 1;
  while (P < k) P <<= 1;
  for (int i = k + tid; i < P; i += kTopkThreads) {
    sel_key[i] = 0;
    sel_idx[i] = 0x7fffffff;
  }
  __syncthreads();
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < P; i += kTopkThreads) {
        const int j = i ^ stride;
        if (j > i) {
          const bool desc = (i & size) == 0;  // first half of each block sorts "best first"
          const unsigned int ka = sel_key[i], kb = sel_key[j];
          const int ia = sel_idx[i], ib = sel_idx[j];
          const bool a_first = ka > kb || (ka == kb && ia < ib);
          if (desc != a_first) {
            sel_key[i] = kb; sel_key[j] = ka;
            sel_idx[i] = ib; sel_idx[j] = ia;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int j = tid; j < k; j += kTopkThreads) {
    const int i = sel_idx[j];
    idx[(long long)b * ld_o + j] = i;
    if (vals) vals[(long long)b * ld_o + j] = row[i];
  }
}

// ------------------------------------------------------------------------------------------
// Gather: out[g, j] = slot row idx[g, j] of the flat library (flat index f -> chunk f / n_flat,
// slot f % n_flat; chunk c lives on page chunk_page[c]) for j < k, zero rows for k <= j < kpad.
// One workgroup per (set g, 4 output rows); 16-byte copies.
__global__ __launch_bounds__(256) void gather_pages_kernel(
    const _Float16* __restrict__ pages, int slots_per_page, long long page_stride, int d,
    const int* __restrict__ chunk_page, int n_chunks, int n_flat, const int* __restrict__ idx,
    long long ld_idx, int k, int kpad, _Float16* __restrict__ out) {
  const int g = blockIdx.y;
  const int j = blockIdx.x * 4 + threadIdx.x / kWave;
  if (j >= kpad) return;
  const int lane = threadIdx.x & (kWave - 1);
  _Float16* dst = out + ((long long)g * kpad + j) * d;
  const _Float16* src = nullptr;
  if (j < k) {
    const int f = idx[(long long)g * ld_idx + j];
    const int c = f / n_flat, n = f % n_flat;
    if (f >= 0 && c < n_chunks && n < slots_per_page)
      src = pages + (long long)chunk_page[c] * page_stride + (long long)n * d;
  }
  for (int e = lane * 8; e < d; e += kWave * 8) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (src) v = *reinterpret_cast<const u32x4*>(src + e);
    *reinterpret_cast<u32x4*>(dst + e) = v;
  }
}

}  // namespace
}  // namespace xenc

using namespace xenc;

extern "C" int xenc_select_scores(const float* q, int B, int n_q, int n_kv, int hd,
                                  const float* keys, int S, const unsigned char* valid, int pool_mean,
                                  float* scores, long long ld_s, void* stream) {
  if (B < 0 || n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0 || hd <= 0 || S < 0 || ld_s < S ||
      B > 65535)
    return XENC_EINVAL;
  if (B == 0 || S == 0) return XENC_OK;
  if (!q || !keys || !scores) return XENC_ENULL;
  hipLaunchKernelGGL(select_scores_kernel, dim3((S + 3) / 4, B), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), q, n_q, n_kv, hd, keys, S, valid,
                     pool_mean, scores, ld_s);
  return check_launch();
}

extern "C" int xenc_topk_rows(const float* scores, long long ld_s, int B, int S, int k, int* idx,
                              float* vals, long long ld_o, void* stream) {
  if (B < 0 || S < 0 || k < 0 || k > S || k > kTopkMax || ld_s < S || ld_o < k) return XENC_EINVAL;
  if (B == 0 || k == 0) return XENC_OK;
  if (!scores || !idx) return XENC_ENULL;
  hipLaunchKernelGGL(topk_rows_kernel, dim3(B), dim3(kTopkThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), scores, ld_s, S, k, idx, vals, ld_o);
  return check_launch();
}

extern "C" int xenc_gather_pages(const void* pages, int slots_per_page, long long page_stride, int d,
                                 const int* chunk_page, int n_chunks, int n_flat, const int* idx,
                                 long long ld_idx, int G, int k, int kpad, void* out, void* stream) {
  if (slots_per_page <= 0 || d <= 0 || d % 8 != 0 || page_stride < (long long)slots_per_page * d ||
      page_stride % 8 != 0 || n_chunks <= 0 || n_flat <= 0 || G < 0 || k < 0 || kpad < k ||
      ld_idx < k || G > 65535)
    return XENC_EINVAL;
  if (G == 0 || kpad == 0) return XENC_OK;
  if (!pages || !chunk_page || !out || (k > 0 && !idx)) return XENC_ENULL;
  if (!aligned16(pages) || !aligned16(out)) return XENC_EALIGN;
  hipLaunchKernelGGL(gather_pages_kernel, dim3((kpad + 3) / 4, G), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const _Float16*>(pages),
                     slots_per_page, page_stride, d, chunk_page, n_chunks, n_flat, idx, ld_idx, k,
                     kpad, static_cast<_Float16*>(out));
  return check_launch();
}
