// Write-back of the read through the interface's B (the write of the epilogue,
// xenc/injector.py:71-74 and 266-267), for the decode path's few query rows:
//   out[m, o] = row_scale[m] * (sum_k W_g[o, k] r[m, k] + b_g[o]),   g = row_group[m]
// row_scale carries gain_scale * exp(log_gain) * gate per row.  W_g is the fp32 [d_out, d]
// weight of library (depth) g.  This is an HBM-bound skinny GEMM: every W row of a library
// that has rows is streamed from HBM once per 32 of its query rows (once for the decode shapes),
// rows of unused libraries are not read, and the query rows stay in the caches.
//
// Work items are (library with rows, 16 output rows).  Persistent workgroups, as many as the
// CUs hold at once, take the items in turn; each first groups the query rows by library in LDS
// (a counting sort).  The 4 waves of a workgroup take interleaved 32-wide k blocks of an item
// (a k quarter each) and sum their partials in LDS in wave order (deterministic).
//
// Products run on the fp32 matrix cores (v_mfma_f32_16x16x4_f32): W is the A operand (16 output
// rows x 4 k), the query rows the B operand (4 k x 16 rows), up to two 16-row column blocks per
// pass.  A k block travels HBM -> registers -> LDS -> registers: the global loads are
// row-contiguous (8 lanes per 128-byte row segment, two whole cache lines per 16 lanes), each
// wave writes its block to its own padded LDS area and reads it back in the MFMA layout (lane
// q = lane / 16, c = lane % 16 holds row c at k = 32 kb + 16 h + 4 q + (0..3), h = 0, 1; MFMA
// (h, j) takes component j).  Loading the MFMA layout straight from memory would put 16 rows
// in every 16-lane group and cost the L1 one tag lookup per 16 bytes.  A and B agree on the k
// of every lane, so the blocks sum over k in a fixed permuted order.  Loads run two blocks
// ahead of the products, and the last blocks of an item prefetch the next item's first blocks.
#include <algorithm>
#include <mutex>

#include "xenc_common.h"

namespace xenc {
namespace {

constexpr int kWbSplit = 4;         // waves per workgroup = k parts
constexpr int kWbTile = 16;         // output rows per item (one 16-row MFMA tile)
constexpr int kT = kWbTile / 16;    // MFMA tiles per item
constexpr int kWbCols = 16;         // query rows per MFMA column block
constexpr int kWbBlocks = 2;        // column blocks per pass over W (32 query rows)
constexpr int kDepth = 2;           // k blocks in flight per wave
constexpr int kWbMaxRows = 4096;    // query rows per call
constexpr int kWbMaxGroups = 1024;  // libraries per call
typedef float f32x4 __attribute__((ext_vector_type(4)));

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kBufWord3 = 0x00020000;  // raw buffer descriptor word 3 (b128 loads ignore format)
constexpr int kLoadNT = 2;             // nontemporal: each W row is streamed once
constexpr unsigned kOob = 0x80000000u;  // offset past every buffer's end: the load returns 0

// Byte offset of k in a row that starts at row_off, or kOob when k >= d or the row is absent
// (d % 4 == 0: a 4-vector is either whole or past the end).
__device__ __forceinline__ unsigned koff(unsigned row_off, int k, int d) {
  return k < d ? row_off + 4u * (unsigned)k : kOob;
}

template <int AUX>
__device__ __forceinline__ f32x4 load4(__amdgpu_buffer_rsrc_t rsrc, unsigned off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, AUX);
  return __builtin_bit_cast(f32x4, v);
}

// LDS staging area of one wave: a k block of the item's W rows and of up to 32 query rows, rows
// padded to 36 floats (the MFMA-layout reads of 16 rows x 16 bytes then cover all 64 banks).
constexpr int kStride = 36;
constexpr int kStageFloats = (kWbTile + kWbCols * kWbBlocks) * kStride;

// Rows are given as byte offsets into the W and r buffers (kOob for an absent row), for the
// row-contiguous load layout: load instruction i reads rows 8 i + lane / 8.
struct WbRows {
  __amdgpu_buffer_rsrc_t w, r;
  unsigned w_off[kWbTile / 8];              // W rows of load instructions 0..kWbTile/8 - 1
  unsigned x_off[kWbCols * kWbBlocks / 8];  // query rows of load instructions 0..2 NB - 1
};

template <int NB>
__device__ __forceinline__ void wb_load(int kb, int d, int lane, const WbRows& rows,
                                        f32x4 (&w)[kWbTile / 8], f32x4 (&x)[2 * NB]) {
  const int k = kb * 32 + 4 * (lane % 8);
#pragma unroll
  for (int i = 0; i < kWbTile / 8; ++i) w[i] = load4<kLoadNT>(rows.w, koff(rows.w_off[i], k, d));
#pragma unroll
  for (int i = 0; i < 2 * NB; ++i) x[i] = load4<0>(rows.r, koff(rows.x_off[i], k, d));
}

// Operands and outputs of one launch, and the workgroup's row lists in LDS.
struct WbArgs {
  const float* r;
  long long ldr;
  int M, d, d_out, tiles, items;
  const float* W;
  long long wgs, ldw;
  const float* bias;
  long long bgs;
  const float* row_scale;
  float* out;
  long long ldo;
  const int* lib;               // u -> library g (libraries with rows, ascending g)
  const int* start;             // [n_used + 1] first entry of library u in order
  const unsigned short* order;  // rows grouped by u
};

// A unit of work: pass p (query rows 32 p .. 32 p + 31 of library u) of item it = (u, tile).
// nb = 0: no unit.
struct WbUnit {
  int it, p, g, o0, rbase, n, nb;
};

__device__ __forceinline__ WbUnit make_unit(const WbArgs& A, int it, int p) {
  WbUnit x{it, p, 0, 0, 0, 0, 0};
  if (it >= A.items) return x;
  const int u = it / A.tiles;
  const int cnt = A.start[u + 1] - A.start[u];
  x.g = A.lib[u];
  x.o0 = (it % A.tiles) * kWbTile;
  x.rbase = A.start[u] + p * kWbCols * kWbBlocks;
  x.n = min(kWbCols * kWbBlocks, cnt - p * kWbCols * kWbBlocks);
  x.nb = (x.n + kWbCols - 1) / kWbCols;
  return x;
}

__device__ __forceinline__ WbUnit next_unit(const WbArgs& A, const WbUnit& x) {
  const int u = x.it / A.tiles;
  if ((x.p + 1) * kWbCols * kWbBlocks < A.start[u + 1] - A.start[u]) return make_unit(A, x.it, x.p + 1);
  return make_unit(A, x.it + gridDim.x, 0);
}

// Byte sizes fit in 31 bits (checked on the host), so every offset and kOob + k stay apart.
template <int NB>
__device__ __forceinline__ WbRows make_rows(const WbArgs& A, const WbUnit& x, int lane) {
  WbRows rows;
  rows.w = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(A.W + (long long)x.g * A.wgs), 0,
                                             (int)((long long)A.d_out * A.ldw * 4), kBufWord3);
  rows.r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(A.r), 0, (int)((long long)A.M * A.ldr * 4),
                                             kBufWord3);
#pragma unroll
  for (int i = 0; i < kWbTile / 8; ++i) {
    const int o = x.o0 + 8 * i + lane / 8;
    rows.w_off[i] = x.nb > 0 && o < A.d_out ? (unsigned)(o * A.ldw * 4) : kOob;
  }
#pragma unroll
  for (int i = 0; i < kWbCols * kWbBlocks / 8; ++i) {
    const int j = 8 * i + lane / 8;
    rows.x_off[i] = i < 2 * NB && j < x.n ? (unsigned)(A.order[x.rbase + j] * A.ldr * 4) : kOob;
  }
  return rows;
}

// The workgroup's run of consecutive units with NB column blocks.  Each wave takes the k blocks
// wv, wv + 4, ... of a unit; acc[t][b] is the 16 x 16 partial of W tile t against column block
// b (lane holds rows 4q..4q+3, column c).  Loads run D blocks ahead of the products (a ring in
// registers); in a unit's last round the refills fetch the next unit's first blocks, so the
// reduction of one unit overlaps the next unit's first loads.  The loop body has no branch: a
// block past the end loads zeros (its offsets are out of the buffers) and adds zero products,
// so the compiler waits for exactly the oldest block's loads.  Returns with cur = the first
// unit that does not have NB column blocks (or none).
template <int NB, int D>
__device__ __forceinline__ void wb_stream(const WbArgs& A, WbUnit& cur, float* stage, float* red_base,
                                          int wv, int lane) {
  const int nkb = (A.d + 31) / 32;
  const int mine = (nkb - wv + kWbSplit - 1) / kWbSplit;  // k blocks of this wave
  const int rounds = (mine + D - 1) / D;
  const int lr = lane / 8, lc = lane % 8;            // load layout
  const int q = lane / kWbCols, c = lane % kWbCols;  // MFMA layout
  float* sw = stage + wv * kStageFloats;  // W rows 0..kWbTile - 1
  float* sr = sw + kWbTile * kStride;     // query rows 0..16 NB - 1
  f32x4 (*red)[kT * kWbBlocks][kWave] = reinterpret_cast<f32x4 (*)[kT * kWbBlocks][kWave]>(red_base);
  WbRows rows = make_rows<NB>(A, cur, lane);
  f32x4 gw[D][kWbTile / 8], gr[D][2 * NB];
#pragma unroll
  for (int s = 0; s < D; ++s) {
    wb_load<NB>(wv + s * kWbSplit, A.d, lane, rows, gw[s], gr[s]);
    __builtin_amdgcn_sched_barrier(0);  // blocks issue in ring order
  }
  while (true) {
    const WbUnit nxt = next_unit(A, cur);
    const bool chain = nxt.nb == NB;
    const WbRows nrows = make_rows<NB>(A, chain ? nxt : WbUnit{0, 0, cur.g, 0, 0, 0, 0}, lane);
    // The epilogue's operands are loaded now, ahead of the next unit's prefetches: a load
    // issued later would make the epilogue wait for those too (loads complete in order).
    int mrow[NB];
    float sc[NB], bv[kT][4];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int j = b * kWbCols + c;
      mrow[b] = j < cur.n ? A.order[cur.rbase + j] : -1;
      sc[b] = mrow[b] >= 0 && A.row_scale ? A.row_scale[mrow[b]] : 1.f;
    }
#pragma unroll
    for (int t = 0; t < kT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int o = cur.o0 + t * kWbCols + 4 * q + i;
        bv[t][i] = A.bias && o < A.d_out ? A.bias[(long long)cur.g * A.bgs + o] : 0.f;
      }
    f32x4 acc[kT][NB];
#pragma unroll
    for (int t = 0; t < kT; ++t)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[t][b] = f32x4{};
    for (int it = 0; it < rounds; ++it) {
      const bool last = it == rounds - 1;
#pragma unroll
      for (int s = 0; s < D; ++s) {
#pragma unroll
        for (int i = 0; i < kWbTile / 8; ++i)
          *reinterpret_cast<f32x4*>(sw + (8 * i + lr) * kStride + 4 * lc) = gw[s][i];
#pragma unroll
        for (int i = 0; i < 2 * NB; ++i)
          *reinterpret_cast<f32x4*>(sr + (8 * i + lr) * kStride + 4 * lc) = gr[s][i];
        wb_load<NB>(last ? wv + s * kWbSplit : wv + ((it + 1) * D + s) * kWbSplit, A.d, lane,
                    last ? nrows : rows, gw[s], gr[s]);
        __builtin_amdgcn_sched_barrier(0);  // issue the refill here, not after the products
        f32x4 a[kT][2], bq[NB][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int t = 0; t < kT; ++t)
            a[t][h] = *reinterpret_cast<const f32x4*>(sw + (kWbCols * t + c) * kStride + 16 * h + 4 * q);
#pragma unroll
          for (int b = 0; b < NB; ++b)
            bq[b][h] = *reinterpret_cast<const f32x4*>(sr + (kWbCols * b + c) * kStride + 16 * h + 4 * q);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int t = 0; t < kT; ++t)
#pragma unroll
              for (int b = 0; b < NB; ++b)
                acc[t][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][h][j], bq[b][h][j], acc[t][b], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);  // the next block's LDS write waits for its own loads only
      }
    }

    // Sum of the k parts in wave order; wave 0 writes.  Lane (q, c) of tile t, block b holds
    // outputs o0 + 16 t + 4 q + (0..3) of column c.  The partials overwrite the staging areas,
    // so every wave has finished its unit first.
    __syncthreads();
    if (wv > 0) {
#pragma unroll
      for (int t = 0; t < kT; ++t)
#pragma unroll
        for (int b = 0; b < NB; ++b) red[wv - 1][t * NB + b][lane] = acc[t][b];
    }
    __syncthreads();
    if (wv == 0) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (mrow[b] < 0) continue;
#pragma unroll
        for (int t = 0; t < kT; ++t) {
          f32x4 y = acc[t][b];
#pragma unroll
          for (int w = 0; w < kWbSplit - 1; ++w) y += red[w][t * NB + b][lane];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int o = cur.o0 + t * kWbCols + 4 * q + i;
            if (o < A.d_out) A.out[(long long)mrow[b] * A.ldo + o] = (y[i] + bv[t][i]) * sc[b];
          }
        }
      }
    }
    __syncthreads();
    cur = nxt;
    if (!chain) return;
    rows = nrows;
  }
}

// Persistent workgroups: item it = (u, tile) for it = blockIdx.x, + gridDim.x, ... below
// (libraries with rows) x tiles: u-th library that has rows (ascending library index), tile of
// kWbTile output rows; an item has one pass (unit) per 32 of the library's rows.  The grid is
// what the CUs hold at once, so no workgroup waits for a slot.
__global__ __launch_bounds__(kWbSplit * kWave) void write_back_kernel(
    const float* __restrict__ r, long long ldr, int M, int d, const int* __restrict__ row_group,
    int G, const float* __restrict__ W, long long wgs, long long ldw, int d_out,
    const float* __restrict__ bias, long long bgs, const float* __restrict__ row_scale,
    float* __restrict__ out, long long ldo, int tiles) {
  constexpr int kThreads = kWbSplit * kWave;
  __shared__ unsigned short order[kWbMaxRows];  // rows grouped by library (u), see start
  __shared__ int lib[kWbMaxGroups];             // row counts per library g, then u -> g
  __shared__ int uidx[kWbMaxGroups];            // g -> u
  __shared__ int fill[kWbMaxGroups];            // rows of library u placed so far
  __shared__ int start[kWbMaxGroups + 1];       // row counts of library u, then first entries
  __shared__ int wcount[kWbSplit];
  // Staging areas of the waves; after a unit the same memory holds the k-part partials.
  __shared__ __attribute__((aligned(16))) float stage[kWbSplit * kStageFloats];
  static_assert((kWbSplit - 1) * kT * kWbBlocks * kWave * 4 <= kWbSplit * kStageFloats, "partials fit");
  static_assert(kWbMaxRows <= 65536, "row indices are 16-bit");
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  auto group_of = [&](int m) { return min(max(row_group ? row_group[m] : 0, 0), G - 1); };

  // Libraries with rows in ascending order (u -> g), their row counts and the rows grouped by
  // library: an LDS histogram, a ballot compaction of its nonzero entries, a wave scan of the
  // counts, and a scatter of the row indices (the order of rows within a library is free: every
  // row's products and sums are the same in any column of the MFMA tiles).
  for (int g = threadIdx.x; g < G; g += kThreads) {
    lib[g] = 0;
    fill[g] = 0;
  }
  __syncthreads();
  for (int m = threadIdx.x; m < M; m += kThreads) atomicAdd(&lib[group_of(m)], 1);
  __syncthreads();
  constexpr int kPer = kWbMaxGroups / kThreads;
  int cnt_of[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int g = threadIdx.x + i * kThreads;
    cnt_of[i] = g < G ? lib[g] : 0;
  }
  __syncthreads();
  int n_used = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    if (i * kThreads >= G) break;
    const bool f = cnt_of[i] > 0;
    const unsigned long long bal = __ballot(f);
    if (lane == 0) wcount[wv] = __popcll(bal);
    __syncthreads();
    int off = n_used, tot = 0;
#pragma unroll
    for (int w = 0; w < kWbSplit; ++w) {
      off += w < wv ? wcount[w] : 0;
      tot += wcount[w];
    }
    if (f) {
      const int u = off + __popcll(bal & ((1ull << lane) - 1ull));
      const int g = threadIdx.x + i * kThreads;
      lib[u] = g;
      uidx[g] = u;
      start[u] = cnt_of[i];
    }
    n_used += tot;
    __syncthreads();
  }
  if (wv == 0) {  // exclusive scan of the counts
    int carry = 0;
    for (int base = 0; base < n_used; base += kWave) {
      const int i = base + lane;
      const int v = i < n_used ? start[i] : 0;
      int x = v;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int y = __shfl_up(x, o, kWave);
        if (lane >= o) x += y;
      }
      if (i < n_used) start[i] = carry + x - v;
      carry += __shfl(x, kWave - 1, kWave);
    }
    if (lane == 0) start[n_used] = carry;
  }
  __syncthreads();
  for (int m = threadIdx.x; m < M; m += kThreads) {
    const int u = uidx[group_of(m)];
    order[start[u] + atomicAdd(&fill[u], 1)] = (unsigned short)m;
  }
  __syncthreads();

  const WbArgs A{r, ldr, M, d, d_out, tiles, n_used * tiles, W, wgs, ldw, bias, bgs, row_scale,
                 out, ldo, lib, start, order};
  WbUnit cur = make_unit(A, blockIdx.x, 0);
  while (cur.nb > 0) {
    if (cur.nb == 1) wb_stream<1, kDepth>(A, cur, stage, stage, wv, lane);
    else wb_stream<2, kDepth>(A, cur, stage, stage, wv, lane);
  }
}

// Resident workgroups of write_back_kernel on the current device (cached per device).
int write_back_slots(int* slots) {
  static std::mutex mu;
  static int cache[64] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_hip_error(e);
    return XENC_EHIP;
  }
  if (dev < 0 || dev >= 64) return XENC_EINVAL;
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] == 0) {
    int cus = 0, per_cu = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess)
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, write_back_kernel, kWbSplit * kWave, 0);
    if (e != hipSuccess) {
      set_hip_error(e);
      return XENC_EHIP;
    }
    cache[dev] = std::max(1, per_cu) * std::max(1, cus);
  }
  *slots = cache[dev];
  return XENC_OK;
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
  // One library's W and the query rows are addressed by 32-bit buffer offsets.
  if ((long long)d_out * ldw * 4 >= (1LL << 31) || (long long)M * ldr * 4 >= (1LL << 31)) return XENC_EINVAL;
  const long long tiles = (d_out + kWbTile - 1) / kWbTile;
  // At most min(G, M) libraries have rows.  Every CU runs as many workgroups as fit (3 at
  // 4 waves each); the persistent workgroups take the items in turn.
  const long long items = (long long)std::min(G, M) * tiles;
  if (items > 0x7fffffffLL) return XENC_EINVAL;
  int slots = 0;
  if (int rc = write_back_slots(&slots)) return rc;
  const long long grid = std::min<long long>(items, slots);
  hipLaunchKernelGGL(write_back_kernel, dim3((unsigned)grid), dim3(kWbSplit * kWave), 0,
                     reinterpret_cast<hipStream_t>(stream), r, ldr, M, d, row_group, G, W,
                     w_group_stride, ldw, d_out, bias, bias_group_stride, row_scale, out, ldo,
                     (int)tiles);
  return check_launch();
}
