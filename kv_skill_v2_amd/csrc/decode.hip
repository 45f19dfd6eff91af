// Paged split-K decode read of the Library (one or a few query rows per library).
//
// Math (xenc/injector.py:239-265, softmax mode):
//   s[c,n] = <q, K[c,n]>;  p = softmax_n(read_temp * s) over the valid slots of chunk c
//   r      = sum_c w[c] * sum_n p[c,n] K[c,n]          (V = K, tied)
// Only the routed chunks are read: the reference multiplies the other chunks by w = 0.
//
// Work unit = (query m, routed chunk j, slot split s) -> one workgroup of NW waves.
// Layout per wave: lane owns 8 consecutive dims of each 512-dim column block (CB blocks cover
// d), so one slot row of d fp16 values is read by the wave as CB coalesced 1 KiB
// global_load_dwordx4 instructions.  A wave takes SPT slots per step (SPT * CB 16-byte loads in
// flight per lane), forms the SPT partial dots, finishes them with an xor reduce-scatter
// (SPT-1 + log2(64/SPT) shuffles for SPT dots) and broadcasts the SPT scores with readlane.
// The same registers then feed the value accumulation, so each slot row crosses HBM once for
// both the score and the value.  Each wave keeps its own online-softmax state (max, sum,
// acc[8*CB]); the NW waves merge through LDS at the end and the workgroup writes one partial
// (acc[d], max, sum).  A second kernel merges the splits of each routed chunk by log-sum-exp,
// scales each chunk by w[j] / l_j and sums the chunks in a fixed order (deterministic).
#include "xenc_common.h"

namespace xenc {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

// Reduce SPT per-lane partial values over the 64 lanes.  On return v[0] holds, in every lane,
// the full sum for slot j = lane / (64 / SPT).
template <int SPT>
__device__ __forceinline__ void wave_reduce_scatter(float (&v)[SPT], int lane) {
  static_assert(SPT >= 1 && SPT <= 64 && (SPT & (SPT - 1)) == 0, "SPT must be a power of 2");
  int mask = 32;
#pragma unroll
  for (int cnt = SPT; cnt > 1; cnt >>= 1, mask >>= 1) {
    const int half = cnt / 2;
    const bool hi = (lane & mask) != 0;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const float send = hi ? v[i] : v[i + half];
      const float keep = hi ? v[i + half] : v[i];
      v[i] = keep + shfl_xor(send, mask);
    }
  }
#pragma unroll
  for (int mk = 64 / SPT / 2; mk >= 1; mk >>= 1) v[0] += shfl_xor(v[0], mk);
}

template <int CB, int SPT, int NW>
__global__ __launch_bounds__(NW* kWave) void decode_split_kernel(
    const float* __restrict__ q, long long ldq, int d, const _Float16* __restrict__ pages,
    long long page_stride, int slots_per_page, const int* __restrict__ chunk_page,
    const int* __restrict__ chunk_nvalid, const int* __restrict__ chunk_ptr,
    const int* __restrict__ q_group, int G, const int* __restrict__ idx, int kk, int nsplit,
    int split_slots, float scale2, int softmax, float* __restrict__ part_acc,
    float2* __restrict__ part_ml) {
  extern __shared__ float red[];  // [NW][d]
  __shared__ float wml[NW][2];

  const int unit = blockIdx.x;
  const int s = unit % nsplit;
  const int mj = unit / nsplit;
  const int m = mj / kk;
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;

  const int cl = idx[mj];
  const int g = min(max(q_group[m], 0), G - 1);
  const int cbeg = chunk_ptr[g];
  int nv = 0;
  long long pbase = 0;
  if (cl >= 0 && cl < chunk_ptr[g + 1] - cbeg) {  // out-of-range entries read nothing
    const int gc = cbeg + cl;
    nv = min(chunk_nvalid[gc], slots_per_page);
    pbase = (long long)chunk_page[gc] * page_stride;
  }
  const int s0 = s * split_slots;
  const int s1 = min(nv, s0 + split_slots);
  if (s0 >= s1) {  // nothing to read (unrouted entry or a split past the chunk's valid slots)
    if (threadIdx.x == 0) part_ml[unit] = make_float2(-INFINITY, 0.f);
    return;
  }

  float qv[CB][8];
  const float* qrow = q + (long long)m * ldq;
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int d0 = (cb * kWave + lane) * 8;
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
  const _Float16* pg = pages + pbase;

  for (int t0 = s0 + wv * SPT; t0 < s1; t0 += NW * SPT) {
    // Unconditional loads: rows past s1 re-read row s1-1 (excluded below through nval) and
    // columns past d re-read the last 8 columns (their q is 0 and their acc is never stored).
    uint4 kv[SPT][CB];
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      const _Float16* row = pg + (long long)min(t0 + j, s1 - 1) * d;
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
        kv[j][cb] = *reinterpret_cast<const uint4*>(row + min((cb * kWave + lane) * 8, d - 8));
    }
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
    wave_reduce_scatter<SPT>(part, lane);
    float sc[SPT];
#pragma unroll
    for (int j = 0; j < SPT; ++j) sc[j] = readlane(part[0], j * (kWave / SPT));
    const int nval = min(SPT, s1 - t0);

    float coef[SPT];
    if (softmax) {
      float tmax = -INFINITY;
#pragma unroll
      for (int j = 0; j < SPT; ++j)
        if (j < nval) tmax = fmaxf(tmax, sc[j] * scale2);
      const float mnew = fmaxf(mrun, tmax);
      const float alpha = exp2f(mrun - mnew);
      float psum = 0.f;
#pragma unroll
      for (int j = 0; j < SPT; ++j) {
        coef[j] = j < nval ? exp2f(sc[j] * scale2 - mnew) : 0.f;
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
      for (int j = 0; j < SPT; ++j) coef[j] = j < nval ? sc[j] * lin_scale : 0.f;
      lrun = 1.f;
      mrun = 0.f;
    }
    // Keep the tile packed (2 halves per VGPR) between the score and value loops: without this the
    // compiler reuses the fp32 conversions of the score loop and holds 8*CB*SPT floats live.
#pragma unroll
    for (int j = 0; j < SPT; ++j)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
        asm volatile("" : "+v"(kv[j][cb].x), "+v"(kv[j][cb].y), "+v"(kv[j][cb].z),
                     "+v"(kv[j][cb].w));
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

  // Merge the NW waves of this workgroup (fixed order: deterministic).
  if (lane == 0) {
    wml[wv][0] = mrun;
    wml[wv][1] = lrun;
  }
  __syncthreads();
  float mall = -INFINITY;
#pragma unroll
  for (int w = 0; w < NW; ++w)
    if (wml[w][1] > 0.f) mall = fmaxf(mall, wml[w][0]);
  const float wscale = lrun > 0.f ? (softmax ? exp2f(mrun - mall) : 1.f) : 0.f;
  float* myred = red + wv * d;
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int d0 = (cb * kWave + lane) * 8;
    if (d0 < d) {
      *reinterpret_cast<float4*>(myred + d0) =
          make_float4(acc[cb][0] * wscale, acc[cb][1] * wscale, acc[cb][2] * wscale,
                      acc[cb][3] * wscale);
      *reinterpret_cast<float4*>(myred + d0 + 4) =
          make_float4(acc[cb][4] * wscale, acc[cb][5] * wscale, acc[cb][6] * wscale,
                      acc[cb][7] * wscale);
    }
  }
  __syncthreads();
  float* out = part_acc + (long long)unit * d;
  for (int i = threadIdx.x * 4; i < d; i += NW * kWave * 4) {
    float4 t = *reinterpret_cast<const float4*>(red + i);
#pragma unroll
    for (int w = 1; w < NW; ++w) {
      const float4 u = *reinterpret_cast<const float4*>(red + w * d + i);
      t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
    }
    *reinterpret_cast<float4*>(out + i) = t;
  }
  if (threadIdx.x == 0) {
    float lsum = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w)
      if (wml[w][1] > 0.f) lsum += wml[w][1] * (softmax ? exp2f(wml[w][0] - mall) : 1.f);
    part_ml[unit] = make_float2(softmax ? mall : 0.f, lsum);
  }
}

// r[m] = sum_j w_sel[m,j] / l_j * sum_s exp2(m_s - M_j) acc_s   (softmax)
// r[m] = sum_j w_sel[m,j] * sum_s acc_s                          (linear)
__global__ __launch_bounds__(256) void decode_merge_kernel(
    const float* __restrict__ part_acc, const float2* __restrict__ part_ml,
    const int* __restrict__ idx, const float* __restrict__ w_sel, int kk, int nsplit, int d,
    int softmax, float* __restrict__ r, long long ldr) {
  extern __shared__ float coef[];  // [kk * nsplit]
  const int m = blockIdx.x;
  const long long ubase = (long long)m * kk * nsplit;
  for (int j = threadIdx.x; j < kk; j += blockDim.x) {
    const float wj = w_sel[(long long)m * kk + j];
    const bool live = idx[(long long)m * kk + j] >= 0;
    float mj = -INFINITY, lj = 0.f;
    if (live) {
      for (int s = 0; s < nsplit; ++s) {
        const float2 ml = part_ml[ubase + (long long)j * nsplit + s];
        if (ml.y > 0.f) mj = fmaxf(mj, ml.x);
      }
      for (int s = 0; s < nsplit; ++s) {
        const float2 ml = part_ml[ubase + (long long)j * nsplit + s];
        if (ml.y > 0.f) lj += softmax ? ml.y * exp2f(ml.x - mj) : 0.f;
      }
    }
    for (int s = 0; s < nsplit; ++s) {
      const float2 ml = part_ml[ubase + (long long)j * nsplit + s];
      float c = 0.f;
      if (live && ml.y > 0.f) c = softmax ? wj * exp2f(ml.x - mj) / lj : wj;
      coef[j * nsplit + s] = c;
    }
  }
  __syncthreads();
  const int nu = kk * nsplit;
  for (int i = threadIdx.x * 4; i < d; i += blockDim.x * 4) {
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int u = 0; u < nu; ++u) {
      const float c = coef[u];
      if (c != 0.f) {
        const float4 a = *reinterpret_cast<const float4*>(part_acc + (ubase + u) * d + i);
        o.x = fmaf(c, a.x, o.x);
        o.y = fmaf(c, a.y, o.y);
        o.z = fmaf(c, a.z, o.z);
        o.w = fmaf(c, a.w, o.w);
      }
    }
    *reinterpret_cast<float4*>(r + (long long)m * ldr + i) = o;
  }
}

template <int CB>
static void launch_split(dim3 grid, size_t lds, hipStream_t st, const float* q, long long ldq,
                         int d, const _Float16* pages, long long page_stride, int spp,
                         const int* chunk_page, const int* chunk_nvalid, const int* chunk_ptr,
                         const int* q_group, int G, const int* idx, int kk, int nsplit,
                         int split_slots, float scale2, int softmax, float* part_acc,
                         float2* part_ml) {
  constexpr int NW = 4;
  constexpr int SPT = CB <= 4 ? 8 : 4;
  hipLaunchKernelGGL((decode_split_kernel<CB, SPT, NW>), grid, dim3(NW * kWave), lds, st, q, ldq,
                     d, pages, page_stride, spp, chunk_page, chunk_nvalid, chunk_ptr, q_group, G,
                     idx, kk, nsplit, split_slots, scale2, softmax, part_acc, part_ml);
}

static size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace xenc

using namespace xenc;

extern "C" size_t xenc_decode_workspace_bytes(int M, int kk, int nsplit, int d) {
  if (M <= 0 || kk <= 0 || nsplit <= 0 || d <= 0) return 0;
  const size_t units = (size_t)M * kk * nsplit;
  return align256(units * d * sizeof(float)) + align256(units * sizeof(float2));
}

extern "C" int xenc_library_read_decode(const float* q, long long ldq, int M, int d,
                                        const void* pages, int slots_per_page,
                                        long long page_stride, const int* chunk_page,
                                        const int* chunk_nvalid, const int* chunk_ptr,
                                        const int* q_group, int G, const int* idx,
                                        const float* w_sel, int kk, float read_temp, int softmax,
                                        int nsplit, float* r, long long ldr, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  if (M < 0 || d <= 0 || G <= 0 || kk <= 0 || slots_per_page <= 0) return XENC_EINVAL;
  if (d % 8 != 0 || d > 8 * 512) return XENC_EINVAL;
  if (nsplit < 1 || nsplit > 64) return XENC_EINVAL;
  if (ldq < d || ldr < d || ldq % 4 != 0 || ldr % 4 != 0) return XENC_EINVAL;
  if (page_stride < (long long)slots_per_page * d || page_stride % 8 != 0) return XENC_EINVAL;
  if (M == 0) return XENC_OK;
  if (!q || !pages || !chunk_page || !chunk_nvalid || !chunk_ptr || !q_group || !idx || !w_sel ||
      !r || !workspace)
    return XENC_ENULL;
  if (!aligned16(q) || !aligned16(pages) || !aligned16(r) || !aligned16(workspace))
    return XENC_EALIGN;
  if (workspace_bytes < xenc_decode_workspace_bytes(M, kk, nsplit, d)) return XENC_EWORKSPACE;
  const long long units = (long long)M * kk * nsplit;
  if (units > 0x7fffffffLL) return XENC_EINVAL;

  const size_t clds = (size_t)kk * nsplit * sizeof(float);
  if (clds > 64 * 1024) return XENC_EINVAL;
  const size_t units_sz = (size_t)units;
  float* part_acc = static_cast<float*>(workspace);
  float2* part_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) +
                                              align256(units_sz * d * sizeof(float)));
  const int split_slots = (slots_per_page + nsplit - 1) / nsplit;
  const float scale2 = read_temp * kLog2e;
  const _Float16* pg = static_cast<const _Float16*>(pages);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)units);
  const size_t lds = (size_t)4 * d * sizeof(float);
  const int cb = (d + 511) / 512;
  switch (cb) {
#define XENC_CASE(N)                                                                           \
  case N:                                                                                      \
    launch_split<N>(grid, lds, st, q, ldq, d, pg, page_stride, slots_per_page, chunk_page,     \
                    chunk_nvalid, chunk_ptr, q_group, G, idx, kk, nsplit, split_slots, scale2, \
                    softmax, part_acc, part_ml);                                               \
    break;
    XENC_CASE(1) XENC_CASE(2) XENC_CASE(3) XENC_CASE(4)
    XENC_CASE(5) XENC_CASE(6) XENC_CASE(7) XENC_CASE(8)
#undef XENC_CASE
    default:
      return XENC_EINVAL;
  }
  int rc = check_launch();
  if (rc) return rc;
  hipLaunchKernelGGL(decode_merge_kernel, dim3(M), dim3(256), clds, st, part_acc, part_ml, idx,
                     w_sel, kk, nsplit, d, softmax, r, ldr);
  return check_launch();
}
