// Routing kernel: per-query scoring against the library's chunk summary keys, wavefront top-k
// (ties to the lower chunk index) and the softmax over the kept logits.
//
// Follows LibraryInjector.route (xenc/injector.py:220-229):
//   logit = einsum("btd,cd->btc", q, S) * route_temp
//   if top_k and top_k < C: keep topk(top_k), the rest -inf
//   w = softmax(logit, -1)
//
// One workgroup (NW = 8 waves) per query row.  A lane owns float4 columns
// (cb*64 + lane)*4 of the d-long dot product, holds q for them in registers, and each wave
// scores CPI chunks per step (CPI * CB4 float4 loads in flight per lane), so the chunk rows of a
// library stream in parallel instead of one dependent dot at a time.  Each dot is finished
// with a fixed xor-butterfly: the fp32 summation order is the same on every call.  Dots land in
// LDS; wave 0 then selects the top_k (a rank count up to 64 chunks, else wave arg-max rounds).
#include "route_select.h"

namespace xenc {

// Per-row LDS of the top-k: dots | taken | order, ls words each.  ls >= 64 (the rank variant's
// 64 keys of 8 bytes live in taken + order) and a multiple of 4 (16-byte aligned arrays).
__host__ __device__ constexpr int select_lds_stride(int ldw) { return ((ldw > 64 ? ldw : 64) + 3) & ~3; }

// Wave-level top-k (ties -> lower chunk index) and softmax over the kept logits
// (logit = dot * route_temp, ranked and scaled as the reference does).  dots[0..C) hold the raw
// dot products; taken / order are scratch of select_lds_stride(C) words.  Writes the kept weights
// into wrow (which the caller has zeroed), and idx / w_sel rows (-1 / 0 past the kept count).
// Register variant for C <= 64 * R chunks and <= 64 kept: lane l holds chunks l, l + 64, ...;
// each round is a wave argmax (value, then lower index) by xor butterfly, the winner's owner
// retires it, and lane r keeps round r's winner for the softmax.  Same selection and arithmetic
// as the LDS variant below.
template <int R>
__device__ __forceinline__ void select_topk_softmax_reg(const float* dots, int C, int top_k, int kk,
                                        float route_temp, float* wrow, int* irow, float* selrow,
                                        int lane) {
  const bool dense = top_k <= 0 || top_k >= C;
  const int nsel = min(dense ? C : top_k, kk);
  float v[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int c = lane + kWave * i;
    v[i] = c < C ? dots[c] * route_temp : -INFINITY;   // the logit the reference ranks
  }
  int mine_c = -1;        // lane r: chunk chosen in round r
  float mine_v = 0.f;
  if (dense) {            // keep every chunk, in chunk order (nsel = C <= 64 here)
    mine_c = lane < nsel ? lane : -1;
    mine_v = v[0];
  } else {
    for (int r = 0; r < nsel; ++r) {
      float bv = -INFINITY;
      int bc = 0x7fffffff;
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const int c = lane + kWave * i;
        if (c < C && v[i] != -INFINITY && (bc == 0x7fffffff || ranks_before(v[i], c, bv, bc))) {
          bv = v[i];
          bc = c;
        }
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        const float ov = shfl_xor(bv, o);
        const int oc = shfl_xor(bc, o);
        if (oc != 0x7fffffff && (bc == 0x7fffffff || ranks_before(ov, oc, bv, bc))) {
          bv = ov;
          bc = oc;
        }
      }
      if ((bc & (kWave - 1)) == lane) v[bc / kWave] = -INFINITY;   // retire the winner
      if (lane == r) {
        mine_c = bc;
        mine_v = bv;
      }
    }
  }
  // A round finds no candidate only when more than C - nsel logits are -inf: such a slot keeps
  // index -1 and weight 0.
  const bool has = mine_c >= 0 && mine_c < C;
  if (!has && lane < nsel) {
    irow[lane] = -1;
    selrow[lane] = 0.f;
  }
  const float lg = has ? mine_v : -INFINITY;
  const float lmax = wave_max(lg);
  const float e = has ? expf(lg - lmax) : 0.f;
  const float inv = 1.f / wave_sum(e);
  if (has) {
    const float wr = e * inv;
    irow[lane] = mine_c;
    selrow[lane] = wr;
    wrow[mine_c] = wr;
  }
  for (int r = nsel + lane; r < kk; r += kWave) {
    irow[r] = -1;
    selrow[r] = 0.f;
  }
}

__device__ __forceinline__ void select_topk_softmax(float* dots, int* taken, int* order, int C, int top_k,
                                    int kk, float route_temp, float* wrow, int* irow, float* selrow,
                                    int lane) {
  const bool dense = top_k <= 0 || top_k >= C;
  const int nsel = min(dense ? C : top_k, kk);
  if (nsel <= kWave && C <= kWave) {
    select_topk_softmax_rank(dots, reinterpret_cast<unsigned long long*>(taken), C,
                             top_k, kk, route_temp, wrow, irow, selrow, lane);
    return;
  }
  if (nsel <= kWave && C <= 4 * kWave && !dense) {
    select_topk_softmax_reg<4>(dots, C, top_k, kk, route_temp, wrow, irow, selrow, lane);
    return;
  }
  if (dense) {
    for (int r = lane; r < nsel; r += kWave) order[r] = r;
  } else {
    for (int c = lane; c < C; c += kWave) taken[c] = 0;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    for (int r = 0; r < nsel; ++r) {
      float bv = -INFINITY;
      int bc = 0x7fffffff;
      for (int c = lane; c < C; c += kWave) {
        if (!taken[c]) {
          const float v = dots[c] * route_temp;
          if (bc == 0x7fffffff || ranks_before(v, c, bv, bc)) {
            bv = v;
            bc = c;
          }
        }
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        const float ov = shfl_xor(bv, o);
        const int oc = shfl_xor(bc, o);
        if (oc != 0x7fffffff && (bc == 0x7fffffff || ranks_before(ov, oc, bv, bc))) {
          bv = ov;
          bc = oc;
        }
      }
      // bc is the same in every lane; C >= 1 guarantees a candidate exists for r < C.
      if (lane == 0) {
        taken[bc] = 1;
        order[r] = bc;
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();

  float lmax = -INFINITY;
  for (int r = lane; r < nsel; r += kWave) lmax = fmaxf(lmax, dots[order[r]] * route_temp);
  lmax = wave_max(lmax);
  float part = 0.f;
  for (int r = lane; r < nsel; r += kWave) part += expf(dots[order[r]] * route_temp - lmax);
  const float inv = 1.f / wave_sum(part);
  for (int r = lane; r < nsel; r += kWave) {
    const int c = order[r];
    const float wr = expf(dots[c] * route_temp - lmax) * inv;
    irow[r] = c;
    selrow[r] = wr;
    wrow[c] = wr;
  }
  for (int r = nsel + lane; r < kk; r += kWave) {
    irow[r] = -1;
    selrow[r] = 0.f;
  }
}

template <int CB4, int CPI, int NW>
__global__ __launch_bounds__(NW* kWave) void route_topk_kernel(
    const float* __restrict__ q, long long ldq, int d, const float* __restrict__ S,
    const int* __restrict__ chunk_ptr, const int* __restrict__ q_group, int G, int top_k,
    float route_temp, float* __restrict__ w_dense, int ldw, int* __restrict__ idx,
    float* __restrict__ w_sel, int kk) {
  // LDS: dots | taken | order, select_lds_stride(ldw) words each
  extern __shared__ __align__(16) float lds[];
  const int ls = select_lds_stride(ldw);
  float* dots = lds;
  int* taken = reinterpret_cast<int*>(lds + ls);
  int* order = taken + ls;

  const int m = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int g = min(max(q_group[m], 0), G - 1);
  const int c0 = chunk_ptr[g];
  // The dense row has ldw columns: a library with more chunks than that is cut to ldw
  // (the host wrapper rejects such calls before launch; this only keeps memory in bounds).
  const int C = min(chunk_ptr[g + 1] - c0, ldw);
  const float* qrow = q + (long long)m * ldq;

  // Columns past d (last block only) re-read the last float4 with q = 0 there.
  float4 qv[CB4];
#pragma unroll
  for (int cb = 0; cb < CB4; ++cb) {
    const int i = (cb * kWave + lane) * 4;
    qv[cb] = i < d ? *reinterpret_cast<const float4*>(qrow + i) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  for (int cbase = wv; cbase < C; cbase += NW * CPI) {
    float acc[CPI];
#pragma unroll
    for (int u = 0; u < CPI; ++u) {
      const int c = min(cbase + u * NW, C - 1);
      const float* srow = S + (long long)(c0 + c) * d;
      float a = 0.f;
#pragma unroll
      for (int cb = 0; cb < CB4; ++cb) {
        // Summary keys are streamed once per call: nontemporal loads.
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        const f32x4 b = __builtin_nontemporal_load(
            reinterpret_cast<const f32x4*>(srow + min((cb * kWave + lane) * 4, d - 4)));
        a = fmaf(qv[cb].x, b.x, a);
        a = fmaf(qv[cb].y, b.y, a);
        a = fmaf(qv[cb].z, b.z, a);
        a = fmaf(qv[cb].w, b.w, a);
      }
      acc[u] = a;
    }
#pragma unroll
    for (int u = 0; u < CPI; ++u) {
      const float a = wave_sum(acc[u]);
      const int c = cbase + u * NW;
      if (lane == 0 && c < C) dots[c] = a;
    }
  }
  float* wrow = w_dense + (long long)m * ldw;
  for (int c = threadIdx.x; c < ldw; c += NW * kWave) wrow[c] = 0.f;
  __syncthreads();
  if (wv != 0) return;
  select_topk_softmax(dots, taken, order, C, top_k, kk, route_temp, wrow, idx + (long long)m * kk,
                      w_sel + (long long)m * kk, lane);
}


// ------------------------------------------------------------------------------------------
// Routing of many query rows (prefill / registration): rows are grouped by library and the
// q . S dots of a 32-row x 32-chunk tile are one fp32 GEMM tile on MFMA (each summary row is read
// once per 32 query rows instead of once per row).  k steps of 128 are staged through LDS (row
// stride 132 floats) with coalesced loads, the next step's global loads in flight while the
// current step computes; wave w of 8 multiplies columns [16w, 16w + 16) of every step with
// v_mfma_f32_32x32x2f32 (two waves per SIMD: two independent accumulation chains), and the 8
// partial tiles are summed through LDS in wave order.  Workgroup b starts its k-loop at step
// b mod (d / 128) and wraps around: when every workgroup walked its rows from column 0 in step,
// the grid read the same 512-byte window of every q row at once (8192 rows x 32 chunks x d 2048:
// 32.3-32.8 us from column 0, 26.3-26.6 us staggered, both with 8 waves).  The raw
// dots land in w_dense; route_rows_select_kernel then runs the same top-k + softmax as the
// per-row kernel, one wave per row.  Fixed summation order per (row, chunk).  When qh is given,
// the first chunk tile of each row tile also writes the rows it stages as fp16 (qh [M, d]), the
// operand of the MFMA read, so q is read from HBM once for both.
constexpr int kRouteRows = 32, kRouteChunks = 32, kRouteK = 128, kRouteLd = kRouteK + 4;
typedef float f32x4nt __attribute__((ext_vector_type(4)));
constexpr int kRouteThreads = 512;
constexpr int kRouteLoads = kRouteRows * kRouteK / 4 / kRouteThreads;   // float4 per thread per operand

__device__ __forceinline__ int find_tile_group(const int* __restrict__ tile_ptr, int G, int b) {
  int lo = 0, hi = G - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (tile_ptr[mid] <= b) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__global__ __launch_bounds__(kRouteThreads) void route_rows_logits_kernel(
    const float* __restrict__ q, long long ldq, int d, const float* __restrict__ S,
    const int* __restrict__ chunk_ptr, const int* __restrict__ row_ptr,
    const int* __restrict__ tile_ptr, int G, float* __restrict__ w_dense, long long ldw,
    _Float16* __restrict__ qh) {
  __shared__ float lds_rl[(kRouteRows + kRouteChunks) * kRouteLd];   // q rows | S rows; partials
  float* const qs = lds_rl;
  float* const ss = lds_rl + kRouteRows * kRouteLd;
  const int b = blockIdx.x;
  const int g = find_tile_group(tile_ptr, G, b);
  const int rbeg = row_ptr[g], rend = row_ptr[g + 1];
  const int c0 = chunk_ptr[g];
  const int C = min(chunk_ptr[g + 1] - c0, (int)ldw);
  const int nct = (C + kRouteChunks - 1) / kRouteChunks;
  const int local = b - tile_ptr[g];
  const int row0 = rbeg + (local / nct) * kRouteRows;
  const int cb0 = (local % nct) * kRouteChunks;
  const int tid = threadIdx.x;
  // Staging: 32 rows x 32 float4 per k step, kRouteLoads per thread and operand (rows / chunks
  // past the end re-read the last one; their dots are not stored).
  const float* qsrc[kRouteLoads];
  const float* ssrc[kRouteLoads];
  int lrow[kRouteLoads], lk[kRouteLoads];
#pragma unroll
  for (int i = 0; i < kRouteLoads; ++i) {
    const int id = tid + kRouteThreads * i;
    lrow[i] = id / (kRouteK / 4);
    lk[i] = (id % (kRouteK / 4)) * 4;
    qsrc[i] = q + (long long)min(row0 + lrow[i], rend - 1) * ldq + lk[i];
    ssrc[i] = S + (long long)(c0 + min(cb0 + lrow[i], C - 1)) * d + lk[i];
  }
  // Two register slots: the loads of k-step j go out during the MFMAs of step j - 2, right after
  // the slot's previous contents were stored (8 waves keep 32 KiB of q and S rows in flight per
  // workgroup; four slots measured no faster).  Every step is unconditional, so each slot keeps
  // its registers through the loop: the k-loop runs a multiple of NS steps, and steps past d load
  // clamped addresses and store zeros.  Columns past d (d % 4 == 0, so a float4 is all in or all
  // out) are zeroed at the store the same way, never by a masked load, which the compiler would
  // wait for on the spot.
  constexpr int NS = 2;
  float4 qv[NS][kRouteLoads], sv[NS][kRouteLoads];
  // Loop step v reads k-step kreal(v) = (v + rot) % nreal (v < nreal; later steps are past d).
  const int nreal = (d + kRouteK - 1) / kRouteK;
  const int rot = b % nreal;
  auto kreal = [&](int kv) {
    const int v = kv / kRouteK;
    return v < nreal ? ((v + rot) % nreal) * kRouteK : kv;
  };
  auto load = [&](int slot, int kv) {
    const int k0 = kreal(kv);
#pragma unroll
    for (int i = 0; i < kRouteLoads; ++i) {
      const int k = min(k0, d - 4 - lk[i]);
      qv[slot][i] = __builtin_bit_cast(float4, __builtin_nontemporal_load(reinterpret_cast<const f32x4nt*>(qsrc[i] + k)));
      sv[slot][i] = *reinterpret_cast<const float4*>(ssrc[i] + k);
    }
  };
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const int lane = tid & (kWave - 1), wv = tid / kWave;
  const int l32 = lane & 31, hl = lane >> 5;
  const bool write_h = qh != nullptr && cb0 == 0;
  f32x16 acc = {};
  // One k-step from register slot `slot` (a constant after inlining).
  auto step = [&](int slot, int kv) {
    const int k0 = kreal(kv);
    __syncthreads();   // the previous step's LDS reads are done
#pragma unroll
    for (int i = 0; i < kRouteLoads; ++i) {
      const bool in = k0 + lk[i] < d;
      const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 a = in ? qv[slot][i] : z, b = in ? sv[slot][i] : z;
      *reinterpret_cast<float4*>(&qs[lrow[i] * kRouteLd + lk[i]]) = a;
      *reinterpret_cast<float4*>(&ss[lrow[i] * kRouteLd + lk[i]]) = b;
      const int row = row0 + lrow[i];
      if (write_h && in && row < rend) {
        typedef _Float16 half4 __attribute__((ext_vector_type(4)));
        const half4 h = {(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w};
        __builtin_nontemporal_store(h, reinterpret_cast<half4*>(qh + (long long)row * d + k0 + lk[i]));
      }
    }
    __syncthreads();
    load(slot, kv + NS * kRouteK);   // this slot is stored: refill it NS steps ahead
    // Lane l feeds row / chunk l % 32 and columns kb + 4 (l / 32) .. + 3 to four MFMAs: MFMA i
    // contracts column kb + 4h + i of both operands for lane half h.
    constexpr int kPerWave = kRouteK / (kRouteThreads / kWave);
#pragma unroll
    for (int kq = 0; kq < kPerWave; kq += 8) {
      const int kb = wv * kPerWave + kq + hl * 4;
      const f32x4 a = *reinterpret_cast<const f32x4*>(&qs[l32 * kRouteLd + kb]);
      const f32x4 b = *reinterpret_cast<const f32x4*>(&ss[l32 * kRouteLd + kb]);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[i], acc, 0, 0, 0);
    }
  };
#pragma unroll
  for (int j = 0; j < NS; ++j) load(j, j * kRouteK);
  for (int k0 = 0; k0 < d; k0 += NS * kRouteK) {
#pragma unroll
    for (int j = 0; j < NS; ++j) step(j, k0 + j * kRouteK);
  }
  // acc[r] = partial dot of row 8(r/4) + 4hl + r%4, chunk l32.  Sum the 8 waves in order.
  constexpr int NWV = kRouteThreads / kWave;
  static_assert(NWV * 16 * kWave <= (kRouteRows + kRouteChunks) * kRouteLd, "partials fit");
  __syncthreads();
  float* red = lds_rl;
#pragma unroll
  for (int r = 0; r < 16; ++r) red[(wv * 16 + r) * kWave + lane] = acc[r];
  __syncthreads();
  for (int i = tid; i < 16 * kWave; i += kRouteThreads) {
    const int r = i / kWave, ln = i % kWave;
    float v = red[r * kWave + ln];
#pragma unroll
    for (int w = 1; w < NWV; ++w) v += red[(w * 16 + r) * kWave + ln];
    const int row = row0 + (r >> 2) * 8 + (ln >> 5) * 4 + (r & 3);
    const int c = cb0 + (ln & 31);
    if (row < rend && c < C) w_dense[(long long)row * ldw + c] = v;
  }
}

constexpr int kSelectWaves = 4;
constexpr int kSplitRouteRows = 256;   // below this many rows xenc_route_topk splits rows over waves

// Library of row m: q_group[m] (clamped) when given, else the g with row_ptr[g] <= m < row_ptr[g+1].
__global__ __launch_bounds__(kSelectWaves * kWave) void route_rows_select_kernel(
    int M, const int* __restrict__ chunk_ptr, const int* __restrict__ row_ptr,
    const int* __restrict__ q_group, int G, int top_k,
    float route_temp, float* __restrict__ w_dense, int ldw, int* __restrict__ idx,
    float* __restrict__ w_sel, int kk) {
  extern __shared__ __align__(16) float lds[];   // per wave: dots | taken | order, ls words each
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int m = blockIdx.x * kSelectWaves + wv;
  if (m >= M) return;
  const int ls = select_lds_stride(ldw);
  float* dots = lds + (size_t)wv * 3 * ls;
  int* taken = reinterpret_cast<int*>(dots + ls);
  int* order = taken + ls;
  const int g = q_group ? min(max(q_group[m], 0), G - 1)
                        : find_tile_group(row_ptr, G, m);   // row_ptr is non-decreasing: same search
  const int c0 = chunk_ptr[g];
  const int C = min(chunk_ptr[g + 1] - c0, ldw);
  float* wrow = w_dense + (long long)m * ldw;
  for (int c = lane; c < C; c += kWave) dots[c] = wrow[c];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  for (int c = lane; c < ldw; c += kWave) wrow[c] = 0.f;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  select_topk_softmax(dots, taken, order, C, top_k, kk, route_temp, wrow, idx + (long long)m * kk,
                      w_sel + (long long)m * kk, lane);
}


// Few query rows: one wave per (row, two chunks) instead of one workgroup per row, so a handful
// of rows still spreads over the whole GPU.  Each dot uses exactly the per-row kernel's
// arithmetic (lane-owned float4 columns accumulated in block order, then the same xor
// butterfly), so the dots, and hence the routing, are bit-identical to route_topk_kernel's.
// Dots land in w_dense; route_rows_select_kernel (with q_group) finishes.  Grid:
// (M, ceil(ldw / 16)) workgroups of 8 waves; waves whose chunks are past the row's library exit.
template <int CB4>
__global__ __launch_bounds__(8 * kWave) void route_dots_kernel(
    const float* __restrict__ q, long long ldq, int d, const float* __restrict__ S,
    const int* __restrict__ chunk_ptr, const int* __restrict__ q_group, int G,
    float* __restrict__ w_dense, int ldw) {
  // Workgroup (m, y) covers chunks 16 y .. 16 y + 15 of row m: wave w forms the dots of chunks
  // 16 y + w and 16 y + w + 8 from one round of loads (each summed as route_dot_wave sums it).
  const int m = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  const int c = blockIdx.y * 16 + (int)(threadIdx.x / kWave), c2 = c + 8;
  const int g = min(max(q_group[m], 0), G - 1);
  const int c0 = chunk_ptr[g];
  const int C = min(chunk_ptr[g + 1] - c0, ldw);
  if (c >= C) return;   // wave-uniform
  const float* qrow = q + (long long)m * ldq;
  if (c2 < C) {
    const float2 x = route_dot2_wave<CB4>(qrow, S + (long long)(c0 + c) * d, S + (long long)(c0 + c2) * d, d, lane);
    if (lane == 0) {
      w_dense[(long long)m * ldw + c] = x.x;
      w_dense[(long long)m * ldw + c2] = x.y;
    }
  } else {
    const float a = route_dot_wave<CB4>(qrow, S + (long long)(c0 + c) * d, d, lane);
    if (lane == 0) w_dense[(long long)m * ldw + c] = a;
  }
}

int launch_route_select(int M, const int* chunk_ptr, const int* q_group, int G, int top_k,
                        float route_temp, float* w_dense, int ldw, int* idx, float* w_sel, int kk,
                        hipStream_t st) {
  const size_t sel_lds = (size_t)kSelectWaves * 3 * select_lds_stride(ldw) * sizeof(float);
  if (sel_lds > 64 * 1024) return XENC_EINVAL;
  hipLaunchKernelGGL(route_rows_select_kernel, dim3((M + kSelectWaves - 1) / kSelectWaves),
                     dim3(kSelectWaves * kWave), sel_lds, st, M, chunk_ptr, nullptr, q_group, G, top_k,
                     route_temp, w_dense, ldw, idx, w_sel, kk);
  return check_launch();
}

int launch_route_dots(const float* q, long long ldq, int M, int d, const float* S, const int* chunk_ptr,
                      const int* q_group, int G, float* w_dense, int ldw, hipStream_t st) {
  const dim3 grid(M, (unsigned)((ldw + 15) / 16));
  switch ((d + 255) / 256) {
#define XENC_DOTS(N)                                                                             \
  case N:                                                                                        \
    hipLaunchKernelGGL(route_dots_kernel<N>, grid, dim3(8 * kWave), 0, st, q, ldq, d, S,         \
                       chunk_ptr, q_group, G, w_dense, ldw);                                     \
    break;
    XENC_DOTS(1) XENC_DOTS(2) XENC_DOTS(3) XENC_DOTS(4) XENC_DOTS(5) XENC_DOTS(6)
    XENC_DOTS(7) XENC_DOTS(8) XENC_DOTS(9) XENC_DOTS(10) XENC_DOTS(11) XENC_DOTS(12)
    XENC_DOTS(13) XENC_DOTS(14) XENC_DOTS(15) XENC_DOTS(16)
#undef XENC_DOTS
    default:
      return XENC_EINVAL;
  }
  return XENC_OK;
}

}  // namespace xenc

using namespace xenc;

extern "C" int xenc_route_topk(const float* q, long long ldq, int M, int d, const float* S,
                               const int* chunk_ptr, const int* q_group, int G, int top_k,
                               float route_temp, float* w_dense, long long ldw, int* idx,
                               float* w_sel, int kk, void* stream) {
  if (M < 0 || d <= 0 || G <= 0 || kk <= 0 || ldw <= 0) return XENC_EINVAL;
  if (d % 8 != 0 || ldq < d || ldq % 4 != 0) return XENC_EINVAL;
  if (M == 0) return XENC_OK;
  if (!q || !S || !chunk_ptr || !q_group || !w_dense || !idx || !w_sel) return XENC_ENULL;
  if (!aligned16(q) || !aligned16(S)) return XENC_EALIGN;
  if (d > 4096) return XENC_EINVAL;
  const size_t lds = (size_t)select_lds_stride((int)ldw) * 3 * sizeof(float);
  if (ldw > 5460 || lds > 64 * 1024) return XENC_EINVAL;  // up to 5460 chunks per library
  constexpr int NW = 8;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int cb4 = (d + 255) / 256;
  // Fewer rows than about one per CU: one wave per (row, chunk), then the wave top-k per row.
  const size_t sel_lds = (size_t)kSelectWaves * 3 * select_lds_stride((int)ldw) * sizeof(float);
  if (M < kSplitRouteRows && sel_lds <= 64 * 1024) {
    const int rc = launch_route_dots(q, ldq, M, d, S, chunk_ptr, q_group, G, w_dense, (int)ldw, st);
    if (rc != XENC_OK) return rc;
    hipLaunchKernelGGL(route_rows_select_kernel, dim3((M + kSelectWaves - 1) / kSelectWaves),
                       dim3(kSelectWaves * kWave), sel_lds, st, M, chunk_ptr, nullptr, q_group, G,
                       top_k, route_temp, w_dense, (int)ldw, idx, w_sel, kk);
    return check_launch();
  }
  switch (cb4) {
#define XENC_CASE(N)                                                                           \
  case N:                                                                                      \
    hipLaunchKernelGGL((route_topk_kernel<N, (N <= 8 ? 4 : 2), NW>), dim3(M), dim3(NW * kWave), \
                       lds, st, q, ldq, d, S, chunk_ptr, q_group, G, top_k, route_temp,        \
                       w_dense, (int)ldw, idx, w_sel, kk);                                     \
    break;
    XENC_CASE(1) XENC_CASE(2) XENC_CASE(3) XENC_CASE(4) XENC_CASE(5) XENC_CASE(6)
    XENC_CASE(7) XENC_CASE(8) XENC_CASE(9) XENC_CASE(10) XENC_CASE(11) XENC_CASE(12)
    XENC_CASE(13) XENC_CASE(14) XENC_CASE(15) XENC_CASE(16)
#undef XENC_CASE
    default:
      return XENC_EINVAL;
  }
  return check_launch();
}

extern "C" int xenc_route_topk_rows(const float* q, long long ldq, int M, int d, const float* S,
                                    const int* chunk_ptr, const int* row_ptr, const int* tile_ptr,
                                    int G, int n_tiles, int top_k, float route_temp,
                                    float* w_dense, long long ldw, int* idx, float* w_sel, int kk,
                                    void* q_f16, void* stream) {
  if (M < 0 || d <= 0 || G <= 0 || kk <= 0 || ldw <= 0 || n_tiles < 0) return XENC_EINVAL;
  if (d % 8 != 0 || ldq < d || ldq % 4 != 0) return XENC_EINVAL;
  if (ldw > 1364) return XENC_EINVAL;  // up to 1364 chunks per library
  const size_t lds = (size_t)kSelectWaves * 3 * select_lds_stride((int)ldw) * sizeof(float);
  if (M == 0) return XENC_OK;
  if (!q || !S || !chunk_ptr || !row_ptr || !tile_ptr || !w_dense || !idx || !w_sel) return XENC_ENULL;
  if (!aligned16(q) || !aligned16(S)) return XENC_EALIGN;
  if (q_f16 && n_tiles == 0) return XENC_EINVAL;
  if (q_f16 && !aligned16(q_f16)) return XENC_EALIGN;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (n_tiles > 0)
    hipLaunchKernelGGL(route_rows_logits_kernel, dim3(n_tiles), dim3(kRouteThreads), 0, st, q, ldq, d, S,
                       chunk_ptr, row_ptr, tile_ptr, G, w_dense, ldw, static_cast<_Float16*>(q_f16));
  hipLaunchKernelGGL(route_rows_select_kernel, dim3((M + kSelectWaves - 1) / kSelectWaves),
                     dim3(kSelectWaves * kWave), lds, st, M, chunk_ptr, row_ptr, nullptr, G, top_k,
                     route_temp, w_dense, (int)ldw, idx, w_sel, kk);
  return check_launch();
}
