// Prefill / registration read of the Library on MFMA (fp16 operands, fp32 accumulation), and its
// dQ backward.  Many query rows read the same library (a training step or a long prompt), so the
// read is a dense contraction:
//
//   forward   S^T[n, t] = K_c[n] . q_t                 (scores kernel, MFMA, one chunk per tile)
//             p[t, c, n] = softmax_n(read_temp * S)     (epilogue: masked per-chunk softmax)
//             r[t]       = sum_c w[t,c] sum_n p K_c[n]  (readout kernel, MFMA over K^T pages)
//   backward  U^T[n, t] = K_c[n] . g_t                 (scores kernel, MFMA)
//             gamma[t,c] = sum_n p U ;  dS = read_temp * w p (U - gamma)   (epilogue)
//             dq_read[t] = sum_{c,n} dS K_c[n]         (readout kernel)
//             dq_route   = route_temp * sum_c w (dw - sum w dw) S_c, dw = gamma + dL/dw (route bwd)
// This is the math of LibraryInjector._branch (xenc/injector.py:236-265) and of its autograd
// (scripts/register_doc.py:699), with K = V tied.
//
// The scores tile covers a whole chunk (512 slots) x 128 query rows, so the chunk softmax is
// local to the workgroup; Sᵀ is formed (slots as the MFMA M dimension) so that each lane holds 32
// slot scores of 4 query rows: the softmax over slots is an in-lane reduction plus one xor-32
// shuffle plus an 8-wave LDS exchange.  The readout is a plain NT GEMM over the transposed pages
// K^T [d, N] (a one-time copy), so both GEMMs read k-contiguous operands.
#include <algorithm>

#include "xenc_common.h"

namespace xenc {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int BK = 32;              // k (d or slot) columns per main-loop step: two MFMA k16 steps
constexpr int LROW = BK + 8;        // LDS row stride in halves (80 B): conflict-free b128 reads
constexpr int kRowsPerTile = 128;   // query rows per scores tile
constexpr int kSlotsPerTile = 512;  // slots per scores tile (a whole page)

__device__ __forceinline__ f32x16 mfma32(const half8_t& a, const half8_t& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Library g of tile b: tile_ptr[g] <= b < tile_ptr[g+1] (binary search; G is small).
__device__ __forceinline__ int find_group(const int* __restrict__ tile_ptr, int G, int b) {
  int lo = 0, hi = G - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (tile_ptr[mid] <= b) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// ------------------------------------------------------------------------------------------
// fp32 -> fp16 rows: y [M, d] (contiguous) from x [M, ldx].
__global__ void cast_rows_f16_kernel(const float* __restrict__ x, long long ldx, int M, int d,
                                     _Float16* __restrict__ y) {
  const long long n4 = (long long)M * (d / 4);
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n4;
       i += (long long)gridDim.x * blockDim.x) {
    const long long row = i / (d / 4), col = (i % (d / 4)) * 4;
    const float4 v = *reinterpret_cast<const float4*>(x + row * ldx + col);
    half4_t h = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
    *reinterpret_cast<half4_t*>(y + row * d + col) = h;
  }
}

// pages [P, N, d] -> pagesT [P, d, N] through 32x32 LDS tiles.
__global__ __launch_bounds__(256) void transpose_pages_kernel(const _Float16* __restrict__ pages,
                                                              int N, int d,
                                                              _Float16* __restrict__ pagesT) {
  __shared__ _Float16 tile[32][33];
  const long long base = (long long)blockIdx.z * N * d;
  const int d0 = blockIdx.x * 32, n0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int i = ty; i < 32; i += 8) {
    const int n = n0 + i, dd = d0 + tx;
    tile[i][tx] = (n < N && dd < d) ? pages[base + (long long)n * d + dd] : (_Float16)0;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int dd = d0 + i, n = n0 + tx;
    if (dd < d && n < N) pagesT[base + (long long)dd * N + n] = tile[tx][i];
  }
}

// ------------------------------------------------------------------------------------------
// Scores kernel: one workgroup = (library g, 128-row tile, chunk c), 8 waves; wave w owns slots
// [64w, 64w+64) (two 32-row MFMA tiles) x all 128 rows (four 32-column tiles).
// MODE 0 (forward): writes p = masked softmax over the chunk's slots (fp16) into P[t, c*N + n].
// MODE 1 (backward): reads p, writes dS = read_temp * w[t,c] * p * (U - gamma) into dS[t, c*N+n]
//                    and gamma[t, c] = sum_n p U.
template <int MODE>
__global__ __launch_bounds__(512) void scores_kernel(
    const _Float16* __restrict__ X, int d, const int* __restrict__ row_ptr,
    const int* __restrict__ tile_ptr, int G, const _Float16* __restrict__ pages, int N,
    long long page_stride, const int* __restrict__ chunk_ptr, const int* __restrict__ chunk_page,
    const int* __restrict__ chunk_nvalid, float temp, const float* __restrict__ w, long long ldw,
    _Float16* __restrict__ P, long long ldp, _Float16* __restrict__ dS,
    float* __restrict__ gamma, long long ldg) {
  __shared__ _Float16 lA[kSlotsPerTile * LROW];  // K_c tile [512][BK] (+pad)
  __shared__ _Float16 lB[kRowsPerTile * LROW];   // X tile [128][BK] (+pad)
  __shared__ float red[8][kRowsPerTile];          // per-wave row statistics

  const int b = blockIdx.x;
  const int g = find_group(tile_ptr, G, b);
  const int cbeg = chunk_ptr[g];
  const int C = chunk_ptr[g + 1] - cbeg;
  const int local = b - tile_ptr[g];
  const int c = local % C;
  const int rt = local / C;
  const int rbeg = row_ptr[g], rend = row_ptr[g + 1];
  const int row0 = rbeg + rt * kRowsPerTile;
  const int gc = cbeg + c;
  const int nv = min(chunk_nvalid[gc], N);
  const _Float16* K = pages + (long long)chunk_page[gc] * page_stride;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5;   // lane half: k-group of the fragments, +4 row offset of D
  const int l32 = lane & 31;

  // Global -> LDS staging: A is 512 rows x 4 16-byte chunks (4 per thread), B is 128 x 4 (1 each).
  u32x4 ra[4], rb;
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = tid + 512 * i;
      const int row = min(ch >> 2, N - 1);  // rows past N are masked below
      ra[i] = *reinterpret_cast<const u32x4*>(K + (long long)row * d + k0 + (ch & 3) * 8);
    }
    const int xr = min(row0 + (tid >> 2), rend - 1);  // rows past the library are not stored
    rb = *reinterpret_cast<const u32x4*>(X + (long long)xr * d + k0 + (tid & 3) * 8);
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = tid + 512 * i;
      *reinterpret_cast<u32x4*>(lA + (ch >> 2) * LROW + (ch & 3) * 8) = ra[i];
    }
    *reinterpret_cast<u32x4*>(lB + (tid >> 2) * LROW + (tid & 3) * 8) = rb;
  };

  f32x16 acc[2][4];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = (f32x16){};

  gload(0);
  for (int k0 = 0; k0 < d; k0 += BK) {
    __syncthreads();  // previous tile fully consumed
    lstore();
    __syncthreads();
    if (k0 + BK < d) gload(k0 + BK);  // next tile in flight during the MFMAs
#pragma unroll
    for (int ks = 0; ks < BK; ks += 16) {
      half8_t fa[2], fb[4];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
        fa[mt] = *reinterpret_cast<const half8_t*>(lA + (wv * 64 + mt * 32 + l32) * LROW + ks + hl * 8);
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        fb[nt] = *reinterpret_cast<const half8_t*>(lB + (nt * 32 + l32) * LROW + ks + hl * 8);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = mfma32(fa[mt], fb[nt], acc[mt][nt]);
    }
  }

  // acc[mt][nt][r] = S^T[slot][row]: slot = 64w + 32mt + 8(r/4) + 4hl + r%4, row = 32nt + l32.
  auto slot_of = [&](int mt, int r) { return wv * 64 + mt * 32 + (r >> 2) * 8 + hl * 4 + (r & 3); };

  if (MODE == 0) {
    // ---- masked softmax over the chunk's slots, per query row
    float rmax[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      float m = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float v = slot_of(mt, r) < nv ? acc[mt][nt][r] * temp : -INFINITY;
          acc[mt][nt][r] = v;
          m = fmaxf(m, v);
        }
      rmax[nt] = fmaxf(m, shfl_xor(m, 32));
    }
    if (hl == 0)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) red[wv][nt * 32 + l32] = rmax[nt];
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      float m = red[0][nt * 32 + l32];
#pragma unroll
      for (int w2 = 1; w2 < 8; ++w2) m = fmaxf(m, red[w2][nt * 32 + l32]);
      rmax[nt] = m;  // finite: every chunk has >= 1 valid slot
    }
    __syncthreads();
    float rsum[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      float s = 0.f;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = __builtin_amdgcn_exp2f(acc[mt][nt][r] - rmax[nt]);  // exp2(-inf) = 0
          acc[mt][nt][r] = e;
          s += e;
        }
      rsum[nt] = s + shfl_xor(s, 32);
    }
    if (hl == 0)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) red[wv][nt * 32 + l32] = rsum[nt];
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      float s = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < 8; ++w2) s += red[w2][nt * 32 + l32];
      rsum[nt] = 1.f / s;
    }
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int t = row0 + nt * 32 + l32;
      if (t >= rend) continue;
      _Float16* prow = P + (long long)t * ldp + (long long)c * N;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int s0 = slot_of(mt, q4 * 4);
          if (s0 < N) {
            half4_t h = {(_Float16)(acc[mt][nt][q4 * 4 + 0] * rsum[nt]),
                         (_Float16)(acc[mt][nt][q4 * 4 + 1] * rsum[nt]),
                         (_Float16)(acc[mt][nt][q4 * 4 + 2] * rsum[nt]),
                         (_Float16)(acc[mt][nt][q4 * 4 + 3] * rsum[nt])};
            *reinterpret_cast<half4_t*>(prow + s0) = h;
          }
        }
    }
  } else {
    // ---- backward: gamma = sum_n p U, dS = temp * w * p * (U - gamma)
    half4_t pv[2][4][4];
    float gpart[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int t = min(row0 + nt * 32 + l32, rend - 1);
      const _Float16* prow = P + (long long)t * ldp + (long long)c * N;
      float s = 0.f;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int s0 = slot_of(mt, q4 * 4);
          pv[mt][nt][q4] = s0 < N ? *reinterpret_cast<const half4_t*>(prow + s0) : (half4_t){};
#pragma unroll
          for (int e = 0; e < 4; ++e) s += (float)pv[mt][nt][q4][e] * acc[mt][nt][q4 * 4 + e];
        }
      gpart[nt] = s + shfl_xor(s, 32);
    }
    if (hl == 0)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) red[wv][nt * 32 + l32] = gpart[nt];
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      float s = 0.f;
#pragma unroll
      for (int w2 = 0; w2 < 8; ++w2) s += red[w2][nt * 32 + l32];
      gpart[nt] = s;
      const int t = row0 + nt * 32 + l32;
      if (t >= rend) continue;
      if (wv == 0 && hl == 0) gamma[(long long)t * ldg + c] = s;
      const float coef = temp * w[(long long)t * ldw + c];
      _Float16* drow = dS + (long long)t * ldp + (long long)c * N;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int s0 = slot_of(mt, q4 * 4);
          if (s0 < N) {
            half4_t h;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              h[e] = (_Float16)(coef * (float)pv[mt][nt][q4][e] * (acc[mt][nt][q4 * 4 + e] - s));
            *reinterpret_cast<half4_t*>(drow + s0) = h;
          }
        }
    }
  }
}

// ------------------------------------------------------------------------------------------
// Readout kernel: out[t, :] = sum_c scale(t,c) sum_n A[t, c*N + n] K_c[n, :], as an NT GEMM over
// the transposed pages K^T_c [d, N].  Workgroup tile 256 rows x 256 dims, 8 waves (2 x 4), wave
// tile 128 x 64 (4 x 2 MFMA 32x32 tiles).  scale = w[t, c] when w != nullptr (forward read),
// else 1 (the backward dS already carries it).  Rows of one tile belong to one library.
__global__ __launch_bounds__(512) void readout_kernel(
    const _Float16* __restrict__ A, long long lda, const int* __restrict__ row_ptr,
    const int* __restrict__ tile_ptr, int G, const _Float16* __restrict__ pagesT, int N, int d,
    long long page_stride, const int* __restrict__ chunk_ptr, const int* __restrict__ chunk_page,
    const float* __restrict__ w, long long ldw, float* __restrict__ out, long long ldo) {
  __shared__ _Float16 lA[256 * LROW];
  __shared__ _Float16 lB[256 * LROW];

  const int b = blockIdx.x;
  const int g = find_group(tile_ptr, G, b);
  const int local = b - tile_ptr[g];
  const int ntile_d = (d + 255) / 256;
  const int dt = local % ntile_d;
  const int rt = local / ntile_d;
  const int rbeg = row_ptr[g], rend = row_ptr[g + 1];
  const int row0 = rbeg + rt * 256;
  const int d0 = dt * 256;
  const int cbeg = chunk_ptr[g];
  const int C = chunk_ptr[g + 1] - cbeg;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wv >> 2, wn = wv & 3;  // wave tile rows [128wm, +128), dims [64wn, +64)
  const int hl = lane >> 5;
  const int l32 = lane & 31;

  // staging: A 256 rows x 4 chunks (2 per thread), B 256 dims x 4 chunks (2 per thread)
  u32x4 ra[2], rb[2];
  const float* wrow[2];
  const _Float16* arow[2];
  const int ar0 = tid >> 2, ach = tid & 3;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int t = min(row0 + ar0 + 128 * i, rend - 1);
    arow[i] = A + (long long)t * lda;
    wrow[i] = w ? w + (long long)t * ldw : nullptr;
  }
  auto gload = [&](int c, int n0) {
    const long long acol = (long long)c * N + n0 + ach * 8;
    const _Float16* Kt = pagesT + (long long)chunk_page[cbeg + c] * page_stride;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      ra[i] = *reinterpret_cast<const u32x4*>(arow[i] + acol);
      if (w) {
        const _Float16 wh = (_Float16)wrow[i][c];
        half8_t h = __builtin_bit_cast(half8_t, ra[i]);
        const half8_t s = {wh, wh, wh, wh, wh, wh, wh, wh};
        ra[i] = __builtin_bit_cast(u32x4, h * s);
      }
      const int dd = min(d0 + ar0 + 128 * i, d - 1);
      rb[i] = *reinterpret_cast<const u32x4*>(Kt + (long long)dd * N + n0 + ach * 8);
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      *reinterpret_cast<u32x4*>(lA + (ar0 + 128 * i) * LROW + ach * 8) = ra[i];
      *reinterpret_cast<u32x4*>(lB + (ar0 + 128 * i) * LROW + ach * 8) = rb[i];
    }
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = (f32x16){};

  const int ksteps = N / BK;
  const int total = C * ksteps;
  gload(0, 0);
  for (int it = 0; it < total; ++it) {
    __syncthreads();
    lstore();
    __syncthreads();
    if (it + 1 < total) gload((it + 1) / ksteps, ((it + 1) % ksteps) * BK);
#pragma unroll
    for (int ks = 0; ks < BK; ks += 16) {
      half8_t fa[4], fb[2];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
        fa[mt] = *reinterpret_cast<const half8_t*>(lA + (wm * 128 + mt * 32 + l32) * LROW + ks + hl * 8);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
        fb[nt] = *reinterpret_cast<const half8_t*>(lB + (wn * 64 + nt * 32 + l32) * LROW + ks + hl * 8);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = mfma32(fa[mt], fb[nt], acc[mt][nt]);
    }
  }
  // acc[mt][nt][r] = out[row0 + 128wm + 32mt + 8(r/4) + 4hl + r%4][d0 + 64wn + 32nt + l32]
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = row0 + wm * 128 + mt * 32 + (r >> 2) * 8 + hl * 4 + (r & 3);
      if (t >= rend) continue;
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int dd = d0 + wn * 64 + nt * 32 + l32;
        if (dd < d) out[(long long)t * ldo + dd] = acc[mt][nt][r];
      }
    }
}

// ------------------------------------------------------------------------------------------
// Route backward: dq[t] += route_temp * sum_c dl[t,c] S[c], dl = w (dw - sum_c' w dw), for the
// rows t of library g (rows of library g are row_ptr[g] .. row_ptr[g+1]-1).  dw = dw_read
// (+ dw_ext when given).  One workgroup = 16 rows; a thread owns 8 dims.
__global__ __launch_bounds__(256) void route_backward_kernel(
    const float* __restrict__ w, long long ldw, const float* __restrict__ dw_read, long long ldr,
    const float* __restrict__ dw_ext, long long lde, const int* __restrict__ row_ptr,
    const int* __restrict__ rtile_ptr, int G, const float* __restrict__ S,
    const int* __restrict__ chunk_ptr, int d, float route_temp, float* __restrict__ dq,
    long long ldq) {
  constexpr int R = 16;
  extern __shared__ float dl[];  // [R][C]
  const int b = blockIdx.x;
  const int g = find_group(rtile_ptr, G, b);
  const int rbeg = row_ptr[g], rend = row_ptr[g + 1];
  const int row0 = rbeg + (b - rtile_ptr[g]) * R;
  const int cbeg = chunk_ptr[g];
  const int C = chunk_ptr[g + 1] - cbeg;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  // dl for the R rows: wave wv handles rows wv, wv+4, ...
  for (int i = wv; i < R; i += 4) {
    const int t = row0 + i;
    if (t >= rend) continue;
    float sdot = 0.f;
    for (int c = lane; c < C; c += 64) {
      float dv = dw_read[(long long)t * ldr + c];
      if (dw_ext) dv += dw_ext[(long long)t * lde + c];
      sdot += w[(long long)t * ldw + c] * dv;
    }
    sdot = wave_sum(sdot);
    for (int c = lane; c < C; c += 64) {
      float dv = dw_read[(long long)t * ldr + c];
      if (dw_ext) dv += dw_ext[(long long)t * lde + c];
      dl[i * C + c] = route_temp * w[(long long)t * ldw + c] * (dv - sdot);
    }
  }
  __syncthreads();
  for (int d0 = threadIdx.x * 8; d0 < d; d0 += 256 * 8) {
    float acc[R][8];
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[i][e] = 0.f;
    for (int c = 0; c < C; ++c) {
      const float4 s0 = *reinterpret_cast<const float4*>(S + (long long)(cbeg + c) * d + d0);
      const float4 s1 = *reinterpret_cast<const float4*>(S + (long long)(cbeg + c) * d + d0 + 4);
      const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const float f = dl[i * C + c];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[i][e] = fmaf(f, sv[e], acc[i][e]);
      }
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int t = row0 + i;
      if (t >= rend) continue;
      float* o = dq + (long long)t * ldq + d0;
      const float4 a = *reinterpret_cast<const float4*>(o);
      const float4 bq = *reinterpret_cast<const float4*>(o + 4);
      *reinterpret_cast<float4*>(o) =
          make_float4(a.x + acc[i][0], a.y + acc[i][1], a.z + acc[i][2], a.w + acc[i][3]);
      *reinterpret_cast<float4*>(o + 4) =
          make_float4(bq.x + acc[i][4], bq.y + acc[i][5], bq.z + acc[i][6], bq.w + acc[i][7]);
    }
  }
}

}  // namespace xenc

using namespace xenc;

extern "C" int xenc_cast_rows_f16(const float* x, long long ldx, int M, int d, void* y,
                                  void* stream) {
  if (M < 0 || d <= 0 || d % 8 != 0 || ldx < d || ldx % 4 != 0) return XENC_EINVAL;
  if (M == 0) return XENC_OK;
  if (!x || !y) return XENC_ENULL;
  if (!aligned16(x) || !aligned16(y)) return XENC_EALIGN;
  const long long n4 = (long long)M * (d / 4);
  const int blocks = (int)std::min<long long>((n4 + 255) / 256, 4096);
  hipLaunchKernelGGL(cast_rows_f16_kernel, dim3(blocks), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), x, ldx, M, d,
                     static_cast<_Float16*>(y));
  return check_launch();
}

extern "C" int xenc_transpose_pages(const void* pages, int P, int slots_per_page, int d,
                                    void* pages_t, void* stream) {
  if (P < 0 || slots_per_page <= 0 || d <= 0 || d % 8 != 0) return XENC_EINVAL;
  if (P == 0) return XENC_OK;
  if (!pages || !pages_t) return XENC_ENULL;
  if (P > 65535) return XENC_EINVAL;
  const dim3 grid((d + 31) / 32, (slots_per_page + 31) / 32, P);
  hipLaunchKernelGGL(transpose_pages_kernel, grid, dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream),
                     static_cast<const _Float16*>(pages), slots_per_page, d,
                     static_cast<_Float16*>(pages_t));
  return check_launch();
}

static int check_prefill_common(int d, int N, long long page_stride) {
  if (d <= 0 || d % BK != 0) return XENC_EINVAL;          // k loop of the scores kernel
  if (N <= 0 || N > kSlotsPerTile || N % BK != 0) return XENC_EINVAL;  // readout k loop
  if (page_stride < (long long)N * d || page_stride % 8 != 0) return XENC_EINVAL;
  return XENC_OK;
}

extern "C" int xenc_prefill_scores(int mode, const void* x, int d, const int* row_ptr,
                                   const int* tile_ptr, int G, int n_tiles, const void* pages,
                                   int slots_per_page, long long page_stride,
                                   const int* chunk_ptr, const int* chunk_page,
                                   const int* chunk_nvalid, float temp, const float* w,
                                   long long ldw, void* p, long long ldp, void* ds, float* gamma,
                                   long long ldg, void* stream) {
  if (mode != 0 && mode != 1) return XENC_EINVAL;
  if (int rc = check_prefill_common(d, slots_per_page, page_stride)) return rc;
  if (G <= 0 || n_tiles < 0 || ldp % 8 != 0) return XENC_EINVAL;
  if (n_tiles == 0) return XENC_OK;
  if (!x || !row_ptr || !tile_ptr || !pages || !chunk_ptr || !chunk_page || !chunk_nvalid || !p)
    return XENC_ENULL;
  if (mode == 1 && (!w || !ds || !gamma)) return XENC_ENULL;
  if (!aligned16(x) || !aligned16(pages) || !aligned16(p) || (mode == 1 && !aligned16(ds)))
    return XENC_EALIGN;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const _Float16* X = static_cast<const _Float16*>(x);
  const _Float16* pg = static_cast<const _Float16*>(pages);
  if (mode == 0)
    hipLaunchKernelGGL(scores_kernel<0>, dim3(n_tiles), dim3(512), 0, st, X, d, row_ptr, tile_ptr,
                       G, pg, slots_per_page, page_stride, chunk_ptr, chunk_page, chunk_nvalid,
                       temp * kLog2e, w, ldw, static_cast<_Float16*>(p), ldp,
                       static_cast<_Float16*>(ds), gamma, ldg);
  else
    hipLaunchKernelGGL(scores_kernel<1>, dim3(n_tiles), dim3(512), 0, st, X, d, row_ptr, tile_ptr,
                       G, pg, slots_per_page, page_stride, chunk_ptr, chunk_page, chunk_nvalid,
                       temp, w, ldw, static_cast<_Float16*>(p), ldp, static_cast<_Float16*>(ds),
                       gamma, ldg);
  return check_launch();
}

extern "C" int xenc_prefill_readout(const void* a, long long lda, const int* row_ptr,
                                    const int* tile_ptr, int G, int n_tiles, const void* pages_t,
                                    int slots_per_page, int d, long long page_stride,
                                    const int* chunk_ptr, const int* chunk_page, const float* w,
                                    long long ldw, float* out, long long ldo, void* stream) {
  if (int rc = check_prefill_common(d, slots_per_page, page_stride)) return rc;
  if (G <= 0 || n_tiles < 0 || lda % 8 != 0 || ldo < d) return XENC_EINVAL;
  if (n_tiles == 0) return XENC_OK;
  if (!a || !row_ptr || !tile_ptr || !pages_t || !chunk_ptr || !chunk_page || !out)
    return XENC_ENULL;
  if (!aligned16(a) || !aligned16(pages_t)) return XENC_EALIGN;
  hipLaunchKernelGGL(readout_kernel, dim3(n_tiles), dim3(512), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const _Float16*>(a), lda,
                     row_ptr, tile_ptr, G, static_cast<const _Float16*>(pages_t), slots_per_page,
                     d, page_stride, chunk_ptr, chunk_page, w, ldw, out, ldo);
  return check_launch();
}

extern "C" int xenc_route_backward(const float* w, long long ldw, const float* dw_read,
                                   long long ldr, const float* dw_ext, long long lde,
                                   const int* row_ptr, const int* rtile_ptr, int G, int n_tiles,
                                   int cmax, const float* S, const int* chunk_ptr, int d,
                                   float route_temp, float* dq, long long ldq, void* stream) {
  if (d <= 0 || d % 8 != 0 || G <= 0 || n_tiles < 0 || cmax <= 0 || ldq < d || ldq % 4 != 0)
    return XENC_EINVAL;
  if (n_tiles == 0) return XENC_OK;
  if (!w || !dw_read || !row_ptr || !rtile_ptr || !S || !chunk_ptr || !dq) return XENC_ENULL;
  if (!aligned16(S) || !aligned16(dq)) return XENC_EALIGN;
  const size_t lds = (size_t)16 * cmax * sizeof(float);
  if (lds > 64 * 1024) return XENC_EINVAL;
  hipLaunchKernelGGL(route_backward_kernel, dim3(n_tiles), dim3(256), lds,
                     reinterpret_cast<hipStream_t>(stream), w, ldw, dw_read, ldr, dw_ext, lde,
                     row_ptr, rtile_ptr, G, S, chunk_ptr, d, route_temp, dq, ldq);
  return check_launch();
}
