// Routing kernel: per-query scoring against the library's chunk summary keys, wavefront top-k
// (ties to the lower chunk index) and the softmax over the kept logits.
//
// Follows LibraryInjector.route (xenc/injector.py:220-229):
//   logit = einsum("btd,cd->btc", q, S) * route_temp
//   if top_k and top_k < C: keep topk(top_k), the rest -inf
//   w = softmax(logit, -1)
//
// One workgroup per query row.  Each wave takes chunks c = wave, wave + NW, ...; a lane owns
// float4 columns lane, lane+64, ... of the d-long dot product (coalesced 1 KiB per wave load),
// and the dot is finished with a fixed xor-butterfly, so the fp32 summation order is the same
// on every call.  Dots land in LDS; wave 0 then runs top_k rounds of a wave-wide argmax.
#include "xenc_common.h"

namespace xenc {

template <int NW>
__global__ __launch_bounds__(NW* kWave) void route_topk_kernel(
    const float* __restrict__ q, long long ldq, int d, const float* __restrict__ S,
    const int* __restrict__ chunk_ptr, const int* __restrict__ q_group, int G, int top_k,
    float route_temp, float* __restrict__ w_dense, int ldw, int* __restrict__ idx,
    float* __restrict__ w_sel, int kk) {
  // LDS: dots[ldw] fp32 | taken[ldw] int | order[ldw] int
  extern __shared__ float lds[];
  float* dots = lds;
  int* taken = reinterpret_cast<int*>(lds + ldw);
  int* order = taken + ldw;

  const int m = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int g = min(max(q_group[m], 0), G - 1);
  const int c0 = chunk_ptr[g];
  // The dense row has ldw columns: a library with more chunks than that is cut to ldw
  // (the host wrapper rejects such calls before launch; this only keeps memory in bounds).
  const int C = min(chunk_ptr[g + 1] - c0, ldw);
  const float* qrow = q + (long long)m * ldq;

  for (int c = wv; c < C; c += NW) {
    const float* srow = S + (long long)(c0 + c) * d;
    float acc = 0.f;
    for (int i = lane * 4; i < d; i += kWave * 4) {
      const float4 a = *reinterpret_cast<const float4*>(qrow + i);
      const float4 b = *reinterpret_cast<const float4*>(srow + i);
      acc = fmaf(a.x, b.x, acc);
      acc = fmaf(a.y, b.y, acc);
      acc = fmaf(a.z, b.z, acc);
      acc = fmaf(a.w, b.w, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) {
      dots[c] = acc;
      taken[c] = 0;
    }
  }
  float* wrow = w_dense + (long long)m * ldw;
  for (int c = threadIdx.x; c < ldw; c += NW * kWave) wrow[c] = 0.f;
  __syncthreads();
  if (wv != 0) return;

  const bool dense = top_k <= 0 || top_k >= C;
  const int nsel = min(dense ? C : top_k, kk);
  if (dense) {
    for (int r = lane; r < nsel; r += kWave) order[r] = r;
  } else {
    for (int r = 0; r < nsel; ++r) {
      float bv = -INFINITY;
      int bc = 0x7fffffff;
      for (int c = lane; c < C; c += kWave) {
        if (!taken[c]) {
          const float v = dots[c];
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

  // Softmax over the kept logits (logit = dot * route_temp, as the reference scales first).
  float lmax = -INFINITY;
  for (int r = lane; r < nsel; r += kWave) lmax = fmaxf(lmax, dots[order[r]] * route_temp);
  lmax = wave_max(lmax);
  float part = 0.f;
  for (int r = lane; r < nsel; r += kWave) part += expf(dots[order[r]] * route_temp - lmax);
  const float inv = 1.f / wave_sum(part);
  int* irow = idx + (long long)m * kk;
  float* selrow = w_sel + (long long)m * kk;
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
  constexpr int NW = 4;
  const size_t lds = (size_t)ldw * 3 * sizeof(float);
  if (lds > 64 * 1024) return XENC_EINVAL;  // up to 5461 chunks per library
  hipLaunchKernelGGL(route_topk_kernel<NW>, dim3(M), dim3(NW * kWave), lds,
                     reinterpret_cast<hipStream_t>(stream), q, ldq, d, S, chunk_ptr, q_group, G,
                     top_k, route_temp, w_dense, (int)ldw, idx, w_sel, kk);
  return check_launch();
}
