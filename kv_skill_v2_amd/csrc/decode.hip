// Paged split-K decode read of the Library (one or a few query rows per library).
//
// Math (xenc/injector.py:239-265, softmax mode):
//   s[c,n] = <q, K[c,n]>;  p = softmax_n(read_temp * s) over the valid slots of chunk c
//   r      = sum_c w[c] * sum_n p[c,n] K[c,n]          (V = K, tied)
// Only the routed chunks are read: the reference multiplies the other chunks by w = 0.
//
// Work unit = (query m, routed chunk j, slot split s) -> one workgroup of NW waves.
// Layout per wave: lane owns 8 consecutive dims of each 512-dim column block (CB blocks cover
// d), so one slot row of d fp16 values is read by the wave as CB coalesced 1 KiB buffer loads.
// A wave takes SPT slots per step: all SPT*CB 16-byte loads are issued before any is used
// (nontemporal: the pages are streamed once), the SPT partial dots are finished with an xor
// reduce-scatter and broadcast with readlane, and the same registers then feed the value
// accumulation, so each slot row crosses HBM once for both the score and the value.  Each wave
// keeps its own online-softmax state (max, sum, acc[8*CB]); the NW waves merge through LDS and
// the workgroup writes one partial (acc[d], max, sum).
//
// Shared libraries (more query rows than libraries): the (row, routed chunk) entries are first
// ranked by page (page_order_kernel) and the units run in that order, XCD-major: the rows that
// routed the same page then read it on the same XCD at the same time, and all but the first
// reader are served by that XCD's L2.  Partials keep their logical index, so the merge and the
// result do not depend on the order.
//
// Merge (merge_query): the k*nsplit partials of a query are combined by log-sum-exp, chunk j
// scaled by w[j] / l_j, and summed in (j, s) order — a fixed order, so results are
// deterministic.  It runs as a second kernel (merge_kernel), launched after the read: one
// workgroup per query, or for few queries several per query, each summing a slice of the
// columns.  No workgroup of the read waits on a release / acquire or merges on its critical
// path (measured faster than merging in the last-arriving workgroup of each query, for many
// rows and for one).
#include <algorithm>
#include <mutex>

#include "route_select.h"

// Waves per workgroup and slots per wave step (for d <= 2048 / above).  Chosen by measurement:
// large two-pass launches take NW_STREAM waves (the kernel holds 179 VGPRs, two waves per SIMD,
// so two 4-wave workgroups share a CU and one's prologue / tail overlaps the other's streaming:
// B = 64 batched decode 0.197 -> 0.188 ms per step; 64 rows over 8 shared libraries, page-grouped:
// 0.258 -> 0.252 ms per step); small launches (fewer than 256 workgroups) keep NW_WIDE (one row
// x 4 pages: 36.5 against 38.4 us).
#ifndef XENC_DECODE_NW_STREAM
#define XENC_DECODE_NW_STREAM 4
#endif
#ifndef XENC_DECODE_NW_WIDE
#define XENC_DECODE_NW_WIDE 8
#endif
#ifndef XENC_DECODE_SPT
#define XENC_DECODE_SPT 4
#endif
#ifndef XENC_DECODE_SPT_WIDE
#define XENC_DECODE_SPT_WIDE 2
#endif
// Minimum waves per SIMD the compiler must fit the read kernel's registers for (4: two 8-wave
// workgroups per CU).
#ifndef XENC_DECODE_MIN_WAVES
#define XENC_DECODE_MIN_WAVES 1
#endif
// The many-unit 4-wave launches at d <= 2048 step 2 slot rows per wave (8 KiB per wave step at
// d = 2048: the B = 64 batched decode's read 165.1-165.3 against 166.6 us with 4 rows); the
// few-unit 8-wave launches keep XENC_DECODE_SPT.
// Measured and not kept (B = 64 batched decode, same box): two register tiles per wave with the
// next one loading while the current one is consumed (184-185 us, no change; measured again on
// the current kernel: step 182.8 against 175.8 us, the single decode 17.3 against 16.6 us, the
// multi-depth step 251 against 238 us: more loads in flight per wave only lengthen the queues),
// and score dots with q rounded to fp16 through v_dot2_f32_f16 (no faster; moves scores by ~1e-5).

namespace xenc {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Buffer descriptor word 3 for CDNA (raw buffer, 32-bit format fields unused by b128 loads).
constexpr int kBufferWord3 = 0x00020000;
// Cache policy of the page loads: nt (nontemporal).  Streamed reads measured 7.1 TB/s with it
// against 6.2 TB/s without on MI355X.  Pages that more than one entry of a page-grouped run reads
// load with the default policy instead, so that the page stays in L2 for its other readers.
constexpr int kLoadNT = 2;
constexpr int kLoadShared = 0;
// A position of the page order: the entry in the low bits, bit 30 set when other entries read
// the same page.
constexpr int kOrderShared = 1 << 30;

struct DecodeWorkspace {
  int* counters;    // [max_rows] reserved: zeroed once by xenc_decode_workspace_init, unused
  int* order;       // [M * kk]   (row, routed chunk) entries ranked by page (page-grouped runs),
                    //            kOrderShared set when more than one entry reads the page
  float2* part_ml;  // [units]    (max in log2 units, sum) per partial; sum 0 = empty
  float* part_acc;  // [units, d] un-normalised value sums
};

// Routing folded into the read (dots != nullptr): dots [M, ldw] (in the workspace) hold the raw
// q . S dots of every row's chunks (route_dots_kernel), ldw <= 64.  Each workgroup ranks its row's
// chunks itself (select_topk_softmax_rank, the routing kernels' own selection) to find the chunk of
// its routed slot; split 0 of each slot publishes idx / w_sel, and the workgroup of (row, slot 0,
// split 0) writes the row's dense weights into w_dense.
// With S set instead of dots (libraries of at most kDotsInRead chunks), each workgroup also forms
// its row's dots itself, wave w taking chunks w, w + NW, ... with route_dot_wave (the dots of
// route_dots_kernel, bit for bit), so the routing needs no launch of its own.
struct RouteFuse {
  const float* dots;
  float* w_dense;
  int ldw;
  int top_k;
  float route_temp;
  const float* S;
};
constexpr int kDotsInRead = 16;

// LDS of the fused selection: the row's dots (reused for the exponentials), the 64-bit keys,
// the dense weights and the kept (index, weight) list by rank.
struct SelectLds {
  float x[kWave];
  unsigned long long keys[kWave];
  float w[kWave];
  int idx[kWave];
  float sel[kWave];
};

// Dynamic LDS of the read kernel, in floats: the wave merge's rows [NW][d], reused by the
// merge's per-partial lists [4 * kk * nsplit], rounded up to 16 bytes.  Launches with the
// routing folded in add one SelectLds per wave after it; other launches allocate none.
__host__ __device__ inline size_t read_red_floats(int nw, int d, int kk, int nsplit) {
  const size_t tree = (size_t)nw * d;
  const size_t lists = (size_t)4 * kk * nsplit;
  return ((tree > lists ? tree : lists) + 3) & ~size_t(3);
}

// Wave-level: the top-k + softmax of a row from its C dots drow (global or LDS) into sl (dense
// weights zeroed first).
__device__ __forceinline__ void select_row(const RouteFuse& rf, const float* drow, int C, int kk, SelectLds& sl,
                                           int lane) {
  sl.w[lane] = 0.f;
  if (lane < C) sl.x[lane] = drow[lane];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  select_topk_softmax_rank(sl.x, sl.keys, C, rf.top_k, kk, rf.route_temp, sl.w, sl.idx, sl.sel, lane);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Merge the k*nsplit partials of query m into r[m] (run by merge_kernel, or by the last
// workgroup of the query in the in-kernel merge).
// LDS: [m | l | coefficient | unit] per partial (4 * nu words).  Every step is parallel over the
// partials; the value sum runs over the live partials in (chunk, split) order with 8 loads in
// flight, so the result is independent of arrival order.
__device__ void merge_query(const DecodeWorkspace& ws, int m, const int* __restrict__ idx,
                            const float* __restrict__ w_sel, int kk, int nsplit, int d, int softmax,
                            float* __restrict__ r, long long ldr, float* lds, int dlo, int dhi) {
  const int nu = kk * nsplit;
  float* pm = lds;                                        // [nu] partial max (log2 units)
  float* pl = lds + nu;                                   // [nu] partial sum (0 = empty)
  float* coef = lds + 2 * nu;                             // [nu] -> compacted coefficients
  int* unit_of = reinterpret_cast<int*>(lds + 3 * nu);    // [nu] -> compacted partial ids
  __shared__ int nlive;
  const long long ubase = (long long)m * nu;
  for (int u = threadIdx.x; u < nu; u += blockDim.x) {
    const float2 ml = ws.part_ml[ubase + u];
    pm[u] = ml.y > 0.f ? ml.x : -INFINITY;
    pl[u] = ml.y;
  }
  __syncthreads();
  // Coefficient of partial u = (j, s): w_j * 2^(m_s - M_j) / l_j (softmax) or w_j (linear).
  for (int u = threadIdx.x; u < nu; u += blockDim.x) {
    const int j = u / nsplit;
    float c = 0.f;
    if (idx[(long long)m * kk + j] >= 0 && pl[u] > 0.f) {
      const float wj = w_sel[(long long)m * kk + j];
      if (softmax) {
        float mj = -INFINITY, lj = 0.f;
        for (int t = 0; t < nsplit; ++t) mj = fmaxf(mj, pm[j * nsplit + t]);
        for (int t = 0; t < nsplit; ++t) {
          const float lt = pl[j * nsplit + t];
          if (lt > 0.f) lj += lt * __builtin_amdgcn_exp2f(pm[j * nsplit + t] - mj);
        }
        c = wj * __builtin_amdgcn_exp2f(pm[u] - mj) / lj;
      } else {
        c = wj;
      }
    }
    coef[u] = c;
  }
  __syncthreads();
  if (threadIdx.x < kWave) {                             // wave 0: ordered ballot compaction
    int n = 0;
    for (int base = 0; base < nu; base += kWave) {
      const int u = base + (int)threadIdx.x;
      const float c = u < nu ? coef[u] : 0.f;
      const bool live = c != 0.f;
      const unsigned long long mask = __ballot(live);
      const int pos = n + __popcll(mask & ((1ull << threadIdx.x) - 1ull));
      __builtin_amdgcn_wave_barrier();
      if (live) {
        coef[pos] = c;       // pos <= u: never overwrites an entry a later step still reads
        unit_of[pos] = u;
      }
      __builtin_amdgcn_wave_barrier();
      n += __popcll(mask);
    }
    if (threadIdx.x == 0) nlive = n;
  }
  __syncthreads();
  const int n = nlive;
  constexpr int kInFlight = 8;
  for (int i = dlo + threadIdx.x * 4; i < dhi; i += blockDim.x * 4) {
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    int t = 0;
    for (; t + kInFlight <= n; t += kInFlight) {
      float4 a[kInFlight];
#pragma unroll
      for (int k = 0; k < kInFlight; ++k)
        a[k] = *reinterpret_cast<const float4*>(ws.part_acc + (ubase + unit_of[t + k]) * d + i);
#pragma unroll
      for (int k = 0; k < kInFlight; ++k) {
        const float c = coef[t + k];
        o.x = fmaf(c, a[k].x, o.x);
        o.y = fmaf(c, a[k].y, o.y);
        o.z = fmaf(c, a[k].z, o.z);
        o.w = fmaf(c, a[k].w, o.w);
      }
    }
    for (; t < n; ++t) {
      const float c = coef[t];
      const float4 a = *reinterpret_cast<const float4*>(ws.part_acc + (ubase + unit_of[t]) * d + i);
      o.x = fmaf(c, a.x, o.x);
      o.y = fmaf(c, a.y, o.y);
      o.z = fmaf(c, a.z, o.z);
      o.w = fmaf(c, a.w, o.w);
    }
    *reinterpret_cast<float4*>(r + (long long)m * ldr + i) = o;
  }
}

// Per-workgroup constants of the tile loop.
template <int CB>
struct TileCtx {
  __amdgpu_buffer_rsrc_t rsrc;
  int voff[CB];     // byte offset of this lane's 8 columns in a slot row (last block clamped)
  int row_bytes;
  int s1;           // end of this split's valid slots
  float scale2;     // read_temp * log2(e)
  float lin_scale;  // 1 / sqrt(n_valid) (linear read)
  int softmax;
  int lane;
};

// Issue the SPT*CB 16-byte loads of the slot rows t0 .. t0+SPT-1.  Rows past s1 re-read row
// s1-1 (excluded from the softmax through nval) and columns past d re-read the last 8 columns
// (their q is 0 and their acc is never stored).  Nontemporal: pages are streamed once.
template <int SPT, int CB, int AUX = kLoadNT>
__device__ __forceinline__ void load_tile(u32x4 (&kv)[SPT][CB], const TileCtx<CB>& c, int t0) {
#pragma unroll
  for (int j = 0; j < SPT; ++j) {
    const int soff = min(t0 + j, c.s1 - 1) * c.row_bytes;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
      kv[j][cb] = __builtin_amdgcn_raw_buffer_load_b128(c.rsrc, c.voff[cb], soff, AUX);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Score the SPT rows of a loaded tile, update the wave's online softmax and accumulate the
// rows into acc with the same registers (each row is read from HBM once).
template <int SPT, int CB>
__device__ __forceinline__ void consume_tile(u32x4 (&kv)[SPT][CB], const TileCtx<CB>& c, int t0,
                                             const float (&qv)[CB][8], float (&acc)[CB][8],
                                             float& mrun, float& lrun) {
  float part[SPT];
#pragma unroll
  for (int j = 0; j < SPT; ++j) {
    float p = 0.f;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const half8_t h = __builtin_bit_cast(half8_t, kv[j][cb]);
#pragma unroll
      for (int i = 0; i < 8; ++i) p = fmaf(qv[cb][i], (float)h[i], p);
    }
    part[j] = p;
  }
  wave_reduce_scatter<SPT>(part, c.lane);
  float sc[SPT];
#pragma unroll
  for (int j = 0; j < SPT; ++j) sc[j] = readlane(part[0], j * (kWave / SPT));
  const int nval = min(SPT, c.s1 - t0);

  float coef[SPT];
  if (c.softmax) {
    float tmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < SPT; ++j)
      if (j < nval) tmax = fmaxf(tmax, sc[j] * c.scale2);
    const float mnew = fmaxf(mrun, tmax);
    const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
    float psum = 0.f;
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      coef[j] = j < nval ? __builtin_amdgcn_exp2f(sc[j] * c.scale2 - mnew) : 0.f;
      psum += coef[j];
    }
    lrun = lrun * alpha + psum;
    mrun = mnew;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[cb][i] *= alpha;
  } else {
#pragma unroll
    for (int j = 0; j < SPT; ++j) coef[j] = j < nval ? sc[j] * c.lin_scale : 0.f;
    lrun = 1.f;
    mrun = 0.f;
  }
  // Keep the tile packed (2 halves per VGPR) between the score and value loops: without this
  // the compiler reuses the fp32 conversions of the score loop and holds 8*CB*SPT floats live.
#pragma unroll
  for (int j = 0; j < SPT; ++j)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) asm volatile("" : "+v"(kv[j][cb]));
#pragma unroll
  for (int j = 0; j < SPT; ++j) {
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const half8_t h = __builtin_bit_cast(half8_t, kv[j][cb]);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[cb][i] = fmaf(coef[j], (float)h[i], acc[cb][i]);
    }
  }
}

template <int CB, int SPT, int NW>
__global__ __launch_bounds__(NW* kWave, XENC_DECODE_MIN_WAVES) void decode_read_kernel(
    const float* __restrict__ q, long long ldq, int d, const _Float16* __restrict__ pages,
    long long page_stride, int slots_per_page, const int* __restrict__ chunk_page,
    const int* __restrict__ chunk_nvalid, const int* __restrict__ chunk_ptr,
    const int* __restrict__ q_group, int G, int* idx, float* w_sel, int kk, int nsplit,
    int split_slots, float scale2, int softmax, float* __restrict__ r, long long ldr,
    DecodeWorkspace ws, int grouped, RouteFuse rf) {
  // idx / w_sel: read (routed in advance) or written by split 0 of each slot (routing folded in),
  // so neither is declared read-only.
  extern __shared__ __align__(16) float red[];  // [NW][d] wave-merge rows; reused by the merge
  __shared__ float wml[NW][2];
  // One SelectLds per wave after the tree, allocated only when the routing is folded in.
  SelectLds* const sl = reinterpret_cast<SelectLds*>(red + read_red_floats(NW, d, kk, nsplit));

  // Launch position -> logical unit: in page-grouped runs the XCD-major position indexes the
  // page-ranked entries; otherwise the unit is the block index.
  const int pos = grouped ? xcd_remap(blockIdx.x, gridDim.x) : blockIdx.x;
  const int s = pos % nsplit;
  const int word = grouped ? __builtin_amdgcn_readfirstlane(ws.order[pos / nsplit]) : 0;
  const int mj = grouped ? (word & (kOrderShared - 1)) : pos / nsplit;
  const bool shared_page = (word & kOrderShared) != 0;   // workgroup-uniform
  const int unit = mj * nsplit + s;
  const int m = mj / kk;
  const int lane = threadIdx.x & (kWave - 1);
  // Wave index as a provably uniform value, so row offsets stay in SGPRs (buffer soffset).
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);

  const int g = min(max(q_group[m], 0), G - 1);
  const int cbeg = chunk_ptr[g];
  const int C_g = chunk_ptr[g + 1] - cbeg;
  int nv = 0;
  long long pbase = 0;
  if (rf.dots || rf.S) {  // uniform: routing folded into the read
    // Every wave ranks the row's chunks itself (its own LDS, no workgroup barrier) while the
    // valid counts and pages of all the row's chunks load, one per lane; the routed chunk's are
    // then taken from its lane.
    const int j = mj - m * kk;
    const int C = min(C_g, rf.ldw);
    const int lnv = lane < C ? chunk_nvalid[cbeg + lane] : 0;
    const int lpg = lane < C ? chunk_page[cbeg + lane] : 0;
    const float* drow = rf.dots + (long long)m * rf.ldw;
    if (rf.S) {
      __shared__ float row_dots[kDotsInRead];
      // Wave w forms the dots of chunks w, w + NW, ...: two at a time, so both summary rows load
      // in one round trip (each dot summed exactly as route_dot_wave sums it).
      const float* qrow = q + (long long)m * ldq;
      for (int c = wv; c < C; c += 2 * NW) {
        const int c2 = c + NW;
        if (c2 < C) {
          const float2 x = route_dot2_wave<2 * CB>(qrow, rf.S + (long long)(cbeg + c) * d,
                                                   rf.S + (long long)(cbeg + c2) * d, d, lane);
          if (lane == 0) {
            row_dots[c] = x.x;
            row_dots[c2] = x.y;
          }
        } else {
          const float x = route_dot_wave<2 * CB>(qrow, rf.S + (long long)(cbeg + c) * d, d, lane);
          if (lane == 0) row_dots[c] = x;
        }
      }
      __syncthreads();
      drow = row_dots;
    }
    select_row(rf, drow, C, kk, sl[wv], lane);
    const int cl = __builtin_amdgcn_readfirstlane(sl[wv].idx[j]);
    if (cl >= 0 && cl < C) {
      nv = min(__builtin_amdgcn_readlane(lnv, cl), slots_per_page);
      pbase = (long long)__builtin_amdgcn_readlane(lpg, cl) * page_stride;
    }
    if (s == 0 && threadIdx.x == 0) {   // thread 0 stores: its release below covers them
      idx[mj] = cl;
      w_sel[mj] = sl[0].sel[j];
    }
    if (s == 0 && j == 0 && wv == 0)
      for (int c = lane; c < rf.ldw; c += kWave) rf.w_dense[(long long)m * rf.ldw + c] = c < C ? sl[0].w[c] : 0.f;
  } else {
    const int cl = idx[mj];
    if (cl >= 0 && cl < C_g) {  // out-of-range entries read nothing
      const int gc = cbeg + cl;
      nv = min(chunk_nvalid[gc], slots_per_page);
      pbase = (long long)chunk_page[gc] * page_stride;
    }
  }
  const int s0 = s * split_slots;
  const int s1 = min(nv, s0 + split_slots);

  if (s0 < s1) {  // workgroup-uniform: a routed split with valid slots
    float qv[CB][8];
    const float* qrow = q + (long long)m * ldq;
    int voff[CB];  // byte offset of this lane's 8 columns in a slot row (last block clamped)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int d0 = (cb * kWave + lane) * 8;
      voff[cb] = min(d0, d - 8) * 2;
      if (d0 < d) {
        const float4 a = *reinterpret_cast<const float4*>(qrow + d0);
        const float4 b = *reinterpret_cast<const float4*>(qrow + d0 + 4);
        qv[cb][0] = a.x; qv[cb][1] = a.y; qv[cb][2] = a.z; qv[cb][3] = a.w;
        qv[cb][4] = b.x; qv[cb][5] = b.y; qv[cb][6] = b.z; qv[cb][7] = b.w;
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) qv[cb][i] = 0.f;
      }
    }

    float acc[CB][8];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[cb][i] = 0.f;
    float mrun = -INFINITY, lrun = 0.f;
    const float lin_scale = rsqrtf((float)nv);
    // One buffer descriptor per page: loads take a uniform row offset (soffset) plus this
    // lane's column offset, so no 64-bit address is kept per load.
    const __amdgpu_buffer_rsrc_t page_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(pages + pbase), 0, slots_per_page * d * 2, kBufferWord3);
    const int row_bytes = d * 2;

    TileCtx<CB> ctx;
    ctx.rsrc = page_rsrc;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) ctx.voff[cb] = voff[cb];
    ctx.row_bytes = row_bytes;
    ctx.s1 = s1;
    ctx.scale2 = scale2;
    ctx.lin_scale = lin_scale;
    ctx.softmax = softmax;
    ctx.lane = lane;
    // Wave wv takes slot rows first, first + step, ... (SPT rows each) of the split.
    const int step = NW * SPT;
    const int first = s0 + wv * SPT;
    const int ntile = first < s1 ? (s1 - first + step - 1) / step : 0;
    if (shared_page) {
      for (int i = 0; i < ntile; ++i) {
        u32x4 ka[SPT][CB];
        load_tile<SPT, CB, kLoadShared>(ka, ctx, first + i * step);
        consume_tile<SPT, CB>(ka, ctx, first + i * step, qv, acc, mrun, lrun);
      }
    } else {
      for (int i = 0; i < ntile; ++i) {
        u32x4 ka[SPT][CB];
        load_tile<SPT, CB>(ka, ctx, first + i * step);
        consume_tile<SPT, CB>(ka, ctx, first + i * step, qv, acc, mrun, lrun);
      }
    }

    // Merge the NW waves of this workgroup: rescale each wave to the common max, every wave puts
    // its sums in its own LDS row, and each thread adds up its columns over the NW rows in a fixed
    // pairwise order (round h: row i += row i + h, i < h; the order a tree over the waves would
    // use), so the result is deterministic.  One LDS exchange instead of log2(NW) rounds.
    if (lane == 0) {
      wml[wv][0] = mrun;
      wml[wv][1] = lrun;
    }
    __syncthreads();
    float mall = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w)
      if (wml[w][1] > 0.f) mall = fmaxf(mall, wml[w][0]);
    const float wscale = lrun > 0.f ? (softmax ? __builtin_amdgcn_exp2f(mrun - mall) : 1.f) : 0.f;
    {
      float* dst = red + wv * d;
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int d0 = (cb * kWave + lane) * 8;
        if (d0 < d) {
          *reinterpret_cast<float4*>(dst + d0) =
              make_float4(acc[cb][0] * wscale, acc[cb][1] * wscale, acc[cb][2] * wscale, acc[cb][3] * wscale);
          *reinterpret_cast<float4*>(dst + d0 + 4) =
              make_float4(acc[cb][4] * wscale, acc[cb][5] * wscale, acc[cb][6] * wscale, acc[cb][7] * wscale);
        }
      }
    }
    __syncthreads();
    // Thread t sums columns 4t, 4t + 4 NW kWave, ... and stores them as the partial
    // (merge_kernel reads it after this kernel).
    float* const out = ws.part_acc + (long long)unit * d;
    for (int i = threadIdx.x * 4; i < d; i += NW * kWave * 4) {
      float4 v[NW];
#pragma unroll
      for (int w = 0; w < NW; ++w) v[w] = *reinterpret_cast<const float4*>(red + w * d + i);
#pragma unroll
      for (int h = NW / 2; h >= 1; h /= 2)
#pragma unroll
        for (int w = 0; w < h; ++w) {
          v[w].x += v[w + h].x;
          v[w].y += v[w + h].y;
          v[w].z += v[w + h].z;
          v[w].w += v[w + h].w;
        }
      *reinterpret_cast<float4*>(out + i) = v[0];
    }
    if (threadIdx.x == 0) {
      float lsum = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w)
        if (wml[w][1] > 0.f)
          lsum += wml[w][1] * (softmax ? __builtin_amdgcn_exp2f(wml[w][0] - mall) : 1.f);
      ws.part_ml[unit] = make_float2(softmax ? mall : 0.f, lsum);
    }
  } else if (threadIdx.x == 0) {  // nothing to read: an unrouted entry or a split past the tail
    ws.part_ml[unit] = make_float2(-INFINITY, 0.f);
  }

  // The partials are merged by merge_kernel, launched after this kernel: the stream order
  // publishes them, and no workgroup waits on a release / acquire or merges on the critical
  // path.
}

// Page-grouped runs: entry i = (row i / kk, routed chunk i % kk) of the n = M * kk entries gets
// its rank among the entries ordered by (page, i); unrouted entries sort last.  Workgroup b
// ranks entries [64b, 64b + 64): every workgroup builds all n keys in LDS, then 8 threads per
// entry each count the keys before it, thread t of the 8 over keys t, t + 8, ... (the 8 read
// consecutive words: no bank conflict), and a reduction over the 8 adds the counts (integers:
// the order of the adds does not matter).  The same pass counts the entries on the entry's page,
// and entries of a page read more than once are marked (kOrderShared).
constexpr int kOrderMax = 1024;
constexpr int kOrderPerWg = 64;
__global__ __launch_bounds__(512) void page_order_kernel(
    const int* __restrict__ idx, const int* __restrict__ q_group, const int* __restrict__ chunk_ptr,
    const int* __restrict__ chunk_page, int G, int kk, int n, int* __restrict__ order) {
  __shared__ int key[kOrderMax];
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int g = min(max(q_group[i / kk], 0), G - 1);
    const int cbeg = chunk_ptr[g];
    const int cl = idx[i];
    key[i] = (cl >= 0 && cl < chunk_ptr[g + 1] - cbeg) ? chunk_page[cbeg + cl] : 0x7fffffff;
  }
  __syncthreads();
  const int i = blockIdx.x * kOrderPerWg + threadIdx.x / 8;   // the entry this thread helps rank
  const int part = threadIdx.x & 7;
  int cnt = 0, same = 0;
  if (i < n) {
    const int ki = key[i];
#pragma unroll 8
    for (int j = part; j < n; j += 8) {
      const int kj = key[j];
      cnt += (kj < ki || (kj == ki && j < i)) ? 1 : 0;
      same += kj == ki ? 1 : 0;
    }
  }
  cnt = (int)group_sum<8>((float)cnt);   // counts <= 1024: exact in fp32, summed by DPP
  same = (int)group_sum<8>((float)same);
  if (i < n && part == 0) order[cnt] = i | (same > 1 && key[i] != 0x7fffffff ? kOrderShared : 0);
}

// Second pass of a large launch: one workgroup per query row merges its partials (the same
// merge_query, so the result is bit-identical to the in-kernel merge).
__global__ __launch_bounds__(512) void merge_kernel(DecodeWorkspace ws, const int* __restrict__ idx,
                                                    const float* __restrict__ w_sel, int kk,
                                                    int nsplit, int d, int softmax,
                                                    float* __restrict__ r, long long ldr) {
  extern __shared__ float lds[];
  // gridDim.y workgroups share a query row, each summing one slice of its d columns (slice
  // width `slice`, a multiple of 4): for few rows the partials are read by many CUs at once.
  const int slice = ((d + (int)gridDim.y - 1) / (int)gridDim.y + 3) & ~3;
  const int dlo = (int)blockIdx.y * slice;
  merge_query(ws, blockIdx.x, idx, w_sel, kk, nsplit, d, softmax, r, ldr, lds, dlo, min(d, dlo + slice));
}

__global__ void fill_zero_kernel(int* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

static size_t host_align256(size_t x) { return (x + 255) & ~size_t(255); }

// Workspace: [counters: max_rows ints | page order / routing dots: M * max(kk, 64) words |
// (m, l) per partial | acc per partial], each region 256-B aligned.  The second region holds the
// page order of page-grouped runs, or the q . S dots when the routing is folded into the read
// (never both in one call).
// The first region (max_rows ints, zeroed once by xenc_decode_workspace_init) is kept so that the
// layout and the set-up call stay as callers know them; the read no longer counts arrivals in it.
static DecodeWorkspace carve(void* base, int max_rows, int M, int kk, int nsplit) {
  const size_t units = (size_t)M * kk * nsplit;
  char* p = static_cast<char*>(base);
  DecodeWorkspace ws;
  ws.counters = reinterpret_cast<int*>(p);
  p += host_align256((size_t)max_rows * sizeof(int));
  ws.order = reinterpret_cast<int*>(p);
  p += host_align256((size_t)M * std::max(kk, kWave) * sizeof(int));
  ws.part_ml = reinterpret_cast<float2*>(p);
  p += host_align256(units * sizeof(float2));
  ws.part_acc = reinterpret_cast<float*>(p);
  return ws;
}

template <int CB, int NW>
static void launch_read(dim3 grid, size_t lds, hipStream_t st, const float* q, long long ldq,
                        int d, const _Float16* pages, long long page_stride, int spp,
                        const int* chunk_page, const int* chunk_nvalid, const int* chunk_ptr,
                        const int* q_group, int G, const int* idx, const float* w_sel, int kk,
                        int nsplit, int split_slots, float scale2, int softmax, float* r,
                        long long ldr, const DecodeWorkspace& ws, int grouped, const RouteFuse& rf) {
  constexpr int SPT = CB == 4 && NW == XENC_DECODE_NW_STREAM ? 2
                      : CB <= 4                                 ? XENC_DECODE_SPT
                      : CB == 5                                 ? XENC_DECODE_SPT_WIDE
                                                                : 1;
  hipLaunchKernelGGL((decode_read_kernel<CB, SPT, NW>), grid, dim3(NW * kWave), lds, st, q, ldq,
                     d, pages, page_stride, spp, chunk_page, chunk_nvalid, chunk_ptr, q_group, G,
                     const_cast<int*>(idx), const_cast<float*>(w_sel), kk, nsplit, split_slots, scale2,
                     softmax, r, ldr, ws, grouped, rf);
}

// Launches of fewer workgroups than this (few query rows, latency-bound) use 8-wave workgroups,
// larger ones 4-wave workgroups (two per CU).
constexpr long long kWideUnits = 256;

// Workgroups of merge_kernel per query row: for few rows the row's columns are split so that
// about 8 workgroups read the partials side by side (slices of at least 256 columns).  The
// single-sequence decode (1 row, 4 pages x 8 splits) measured 16.6 us per step this way, 17.5 us
// with the merge done by the last-arriving workgroup of the read (one CU reading 32 partials
// behind a device-scope release and an arrival count).
static int merge_slices(int M, int d) {
  const int want = std::max(1, 8 / std::max(M, 1));
  return std::max(1, std::min(want, d / 256));
}

}  // namespace xenc

using namespace xenc;

static size_t workspace_need(int max_rows, long long rows, int kk, long long units, int d) {
  return host_align256((size_t)max_rows * sizeof(int)) +
         host_align256((size_t)rows * std::max(kk, kWave) * sizeof(int)) +
         host_align256(units * sizeof(float2)) + host_align256(units * d * sizeof(float));
}

extern "C" size_t xenc_decode_workspace_bytes(int max_rows, int kk, int nsplit, int d) {
  if (max_rows <= 0 || kk <= 0 || nsplit <= 0 || d <= 0) return 0;
  return workspace_need(max_rows, max_rows, kk, (long long)max_rows * kk * nsplit, d);
}

extern "C" int xenc_decode_workspace_init(void* workspace, size_t workspace_bytes, int max_rows,
                                          void* stream) {
  if (max_rows <= 0) return XENC_EINVAL;
  if (!workspace) return XENC_ENULL;
  if (!aligned16(workspace)) return XENC_EALIGN;
  if (workspace_bytes < (size_t)max_rows * sizeof(int)) return XENC_EWORKSPACE;
  const int blocks = std::min((max_rows + 255) / 256, 1024);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<int*>(workspace), max_rows);
  return check_launch();
}

// Workgroup size and LDS bytes (dynamic, then the whole workgroup's) of a read launch.
static int read_waves(long long units) {
  return units < kWideUnits ? XENC_DECODE_NW_WIDE : XENC_DECODE_NW_STREAM;
}
static size_t read_dynamic_lds(int nw, int d, int kk, int nsplit, bool fold) {
  return read_red_floats(nw, d, kk, nsplit) * sizeof(float) + (fold ? (size_t)nw * sizeof(SelectLds) : 0);
}
static size_t read_total_lds(int nw, int d, int kk, int nsplit, bool fold) {
  // static part: wml[NW][2] and row_dots[kDotsInRead]
  return read_dynamic_lds(nw, d, kk, nsplit, fold) + (size_t)nw * 2 * sizeof(float) + kDotsInRead * sizeof(float);
}

// Every argument check of the decode read, done before anything is launched (the routing
// launches of xenc_route_read_decode included), so a rejected call leaves its outputs untouched.
static int validate_read(const float* q, long long ldq, int M, int d, const void* pages, int slots_per_page,
                         long long page_stride, const int* chunk_page, const int* chunk_nvalid,
                         const int* chunk_ptr, const int* q_group, int G, const int* idx, const float* w_sel,
                         int kk, int nsplit, const float* r, long long ldr, const void* workspace,
                         size_t workspace_bytes, int max_rows, int short_code, bool fold) {
  if (M < 0 || d <= 0 || G <= 0 || kk <= 0 || slots_per_page <= 0) return XENC_EINVAL;
  if (M > max_rows) return short_code;
  if (d % 8 != 0 || d > 8 * 512) return XENC_EINVAL;
  if (nsplit < 1 || nsplit > 64) return XENC_EINVAL;
  if (ldq < d || ldr < d || ldq % 4 != 0 || ldr % 4 != 0) return XENC_EINVAL;
  if (page_stride < (long long)slots_per_page * d || page_stride % 8 != 0) return XENC_EINVAL;
  if ((long long)slots_per_page * d * 2 > 0x7fffffffLL) return XENC_EINVAL;  // buffer range
  if (M == 0) return XENC_OK;
  if (!q || !pages || !chunk_page || !chunk_nvalid || !chunk_ptr || !q_group || !idx || !w_sel ||
      !r || !workspace)
    return XENC_ENULL;
  if (!aligned16(q) || !aligned16(pages) || !aligned16(r) || !aligned16(workspace))
    return XENC_EALIGN;
  const long long units = (long long)M * kk * nsplit;
  if (units > 0x7fffffffLL) return XENC_EINVAL;
  if (workspace_bytes < workspace_need(max_rows, M, kk, units, d)) return short_code;
  if (read_total_lds(read_waves(units), d, kk, nsplit, fold) > device_lds_limit()) return XENC_EINVAL;
  return XENC_OK;
}

// Validation and launches of the decode read over a workspace of workspace_bytes at `workspace`
// whose counter region is sized for max_rows (shared by the entry points below).
static int read_decode(const float* q, long long ldq, int M, int d, const void* pages,
                       int slots_per_page, long long page_stride, const int* chunk_page,
                       const int* chunk_nvalid, const int* chunk_ptr, const int* q_group, int G,
                       const int* idx, const float* w_sel, int kk, float read_temp, int softmax,
                       int nsplit, float* r, long long ldr, void* workspace, size_t workspace_bytes,
                       int max_rows, int short_code, hipStream_t st, const RouteFuse& rf = RouteFuse{}) {
  const bool fold = rf.dots || rf.S;
  const int vrc = validate_read(q, ldq, M, d, pages, slots_per_page, page_stride, chunk_page, chunk_nvalid,
                                chunk_ptr, q_group, G, idx, w_sel, kk, nsplit, r, ldr, workspace,
                                workspace_bytes, max_rows, short_code, fold);
  if (vrc != XENC_OK || M == 0) return vrc;
  const long long units = (long long)M * kk * nsplit;
  // Page-grouped runs when rows share libraries and there are enough entries to matter.
  const long long entries = (long long)M * kk;
  const int grouped = (!fold && M > G && entries >= 128 && entries <= kOrderMax) ? 1 : 0;
  const int nw = read_waves(units);
  const size_t lds = read_dynamic_lds(nw, d, kk, nsplit, fold);

  const DecodeWorkspace ws = carve(workspace, max_rows, M, kk, nsplit);
  const int split_slots = (slots_per_page + nsplit - 1) / nsplit;
  const float scale2 = read_temp * kLog2e;
  const _Float16* pg = static_cast<const _Float16*>(pages);
  if (grouped)
    hipLaunchKernelGGL(page_order_kernel, dim3((unsigned)((entries + kOrderPerWg - 1) / kOrderPerWg)),
                       dim3(512), 0, st, idx, q_group, chunk_ptr, chunk_page, G, kk, (int)entries,
                       ws.order);
  const dim3 grid((unsigned)units);
  const int cb = (d + 511) / 512;
  switch (cb) {
#define XENC_CASE(N)                                                                              \
  case N:                                                                                         \
    if (nw == XENC_DECODE_NW_STREAM)                                                              \
      launch_read<N, XENC_DECODE_NW_STREAM>(grid, lds, st, q, ldq, d, pg, page_stride,            \
                                            slots_per_page, chunk_page, chunk_nvalid, chunk_ptr,  \
                                            q_group, G, idx, w_sel, kk, nsplit, split_slots,      \
                                            scale2, softmax, r, ldr, ws, grouped, rf);     \
    else                                                                                          \
      launch_read<N, XENC_DECODE_NW_WIDE>(grid, lds, st, q, ldq, d, pg, page_stride,              \
                                          slots_per_page, chunk_page, chunk_nvalid, chunk_ptr,    \
                                          q_group, G, idx, w_sel, kk, nsplit, split_slots,        \
                                          scale2, softmax, r, ldr, ws, grouped, rf);       \
    break;
    XENC_CASE(1) XENC_CASE(2) XENC_CASE(3) XENC_CASE(4)
    XENC_CASE(5) XENC_CASE(6) XENC_CASE(7) XENC_CASE(8)
#undef XENC_CASE
    default:
      return XENC_EINVAL;
  }
  hipLaunchKernelGGL(merge_kernel, dim3(M, merge_slices(M, d)), dim3(512), (size_t)4 * kk * nsplit * sizeof(float),
                     st, ws, idx, w_sel, kk, nsplit, d, softmax, r, ldr);
  return check_launch();
}

extern "C" int xenc_library_read_decode(const float* q, long long ldq, int M, int d,
                                        const void* pages, int slots_per_page,
                                        long long page_stride, const int* chunk_page,
                                        const int* chunk_nvalid, const int* chunk_ptr,
                                        const int* q_group, int G, const int* idx,
                                        const float* w_sel, int kk, float read_temp, int softmax,
                                        int nsplit, float* r, long long ldr, void* workspace,
                                        size_t workspace_bytes, int max_rows, void* stream) {
  return read_decode(q, ldq, M, d, pages, slots_per_page, page_stride, chunk_page, chunk_nvalid,
                     chunk_ptr, q_group, G, idx, w_sel, kk, read_temp, softmax, nsplit, r, ldr,
                     workspace, workspace_bytes, max_rows, XENC_EWORKSPACE,
                     reinterpret_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------- the allocation-free variant
// A file-scope device array replaces the caller's workspace: every GPU the library runs on holds
// its own copy (XENC_DECODE_SCRATCH_BYTES) until the process ends.  In host code `scratch` is
// only a stand-in for the symbol; its device address is looked up once per device with
// hipGetSymbolAddress (with that device current) and only that address reaches kernels.
// The workspace layout is carved for kScratchRows rows; its first (reserved) region is zeroed by
// a kernel the first time a device is used, as xenc_decode_workspace_init does for a caller's.
static __device__ __align__(256) unsigned char scratch[XENC_DECODE_SCRATCH_BYTES];
constexpr int kScratchRows = XENC_DECODE_SCRATCH_ROWS;
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

static int scratch_for_current_device(hipStream_t st, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return XENC_EINVAL;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_hip_error(e);
      return XENC_EHIP;
    }
    hipLaunchKernelGGL(fill_zero_kernel, dim3((kScratchRows + 255) / 256), dim3(256), 0, st,
                       static_cast<int*>(p), kScratchRows);
    const int rc = check_launch();
    if (rc != XENC_OK) return rc;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return XENC_OK;
}

extern "C" int xenc_library_read_decode_noalloc(const float* q, long long ldq, int M, int d,
                                                const void* pages, int slots_per_page,
                                                long long page_stride, const int* chunk_page,
                                                const int* chunk_nvalid, const int* chunk_ptr,
                                                const int* q_group, int G, const int* idx,
                                                const float* w_sel, int kk, float read_temp,
                                                int softmax, int nsplit, float* r, long long ldr,
                                                void* stream) {
  if (M < 0 || d <= 0 || G <= 0 || kk <= 0 || slots_per_page <= 0 || nsplit < 1) return XENC_EINVAL;
  if (M > kScratchRows) return XENC_ESCRATCH;
  if (M == 0) return XENC_OK;
  const long long units = (long long)M * kk * nsplit;
  if (workspace_need(kScratchRows, M, kk, units, d) > (size_t)XENC_DECODE_SCRATCH_BYTES)
    return XENC_ESCRATCH;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  void* ws = nullptr;
  const int rc = scratch_for_current_device(st, &ws);
  if (rc != XENC_OK) return rc;
  return read_decode(q, ldq, M, d, pages, slots_per_page, page_stride, chunk_page, chunk_nvalid,
                     chunk_ptr, q_group, G, idx, w_sel, kk, read_temp, softmax, nsplit, r, ldr, ws,
                     (size_t)XENC_DECODE_SCRATCH_BYTES, kScratchRows, XENC_ESCRATCH, st);
}

// ---------------------------------------------------------------- routing + read in one call
extern "C" int xenc_route_read_decode(const float* q, long long ldq, int M, int d, const float* S,
                                      const void* pages, int slots_per_page, long long page_stride,
                                      const int* chunk_page, const int* chunk_nvalid,
                                      const int* chunk_ptr, const int* q_group, int G, int top_k,
                                      float route_temp, float* w_dense, long long ldw, int* idx,
                                      float* w_sel, int kk, float read_temp, int softmax, int nsplit,
                                      float* r, long long ldr, void* workspace,
                                      size_t workspace_bytes, int max_rows, void* stream) {
  if (M < 0 || d <= 0 || G <= 0 || kk <= 0 || ldw <= 0) return XENC_EINVAL;
  if (M == 0) return XENC_OK;
  if (!S || !w_dense || !idx || !w_sel) return XENC_ENULL;
  if (!aligned16(S)) return XENC_EALIGN;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const long long entries = (long long)M * kk;
  // The read ranks a row's chunks itself when a library has at most 64 and the rows do not share
  // libraries enough for the page-grouped order (which needs the routed chunks before the read),
  // and when the workgroup's LDS then fits the device.
  const bool fold = ldw <= kWave && kk <= kWave && !(M > G && entries >= 128 && entries <= kOrderMax) &&
                    read_total_lds(read_waves(entries * std::max(nsplit, 1)), d, kk, std::max(nsplit, 1), true) <=
                        device_lds_limit();
  // All of the read's checks come first: nothing is launched for a call the read would reject.
  const int vrc = validate_read(q, ldq, M, d, pages, slots_per_page, page_stride, chunk_page, chunk_nvalid,
                                chunk_ptr, q_group, G, idx, w_sel, kk, nsplit, r, ldr, workspace,
                                workspace_bytes, max_rows, XENC_EWORKSPACE, fold);
  if (vrc != XENC_OK) return vrc;
  if (!fold) {
    const int rc = xenc_route_topk(q, ldq, M, d, S, chunk_ptr, q_group, G, top_k, route_temp, w_dense, ldw,
                                   idx, w_sel, kk, stream);
    if (rc != XENC_OK) return rc;
    return read_decode(q, ldq, M, d, pages, slots_per_page, page_stride, chunk_page, chunk_nvalid,
                       chunk_ptr, q_group, G, idx, w_sel, kk, read_temp, softmax, nsplit, r, ldr,
                       workspace, workspace_bytes, max_rows, XENC_EWORKSPACE, st);
  }
  if (ldw <= kDotsInRead) {   // the read's workgroups form the dots too
    const RouteFuse rf{nullptr, w_dense, (int)ldw, top_k, route_temp, S};
    return read_decode(q, ldq, M, d, pages, slots_per_page, page_stride, chunk_page, chunk_nvalid, chunk_ptr,
                       q_group, G, idx, w_sel, kk, read_temp, softmax, nsplit, r, ldr, workspace,
                       workspace_bytes, max_rows, XENC_EWORKSPACE, st, rf);
  }
  float* dots = reinterpret_cast<float*>(carve(workspace, max_rows, M, kk, nsplit).order);
  const int rc = launch_route_dots(q, ldq, M, d, S, chunk_ptr, q_group, G, dots, (int)ldw, st);
  if (rc != XENC_OK) return rc;
  const RouteFuse rf{dots, w_dense, (int)ldw, top_k, route_temp, nullptr};
  return read_decode(q, ldq, M, d, pages, slots_per_page, page_stride, chunk_page, chunk_nvalid, chunk_ptr,
                     q_group, G, idx, w_sel, kk, read_temp, softmax, nsplit, r, ldr, workspace,
                     workspace_bytes, max_rows, XENC_EWORKSPACE, st, rf);
}
