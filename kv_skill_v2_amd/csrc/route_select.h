// Pieces of the routing shared by the routing kernels (route.hip) and the read kernel's fused
// routing prologue (decode.hip): the rank-count top-k + softmax over at most 64 chunks, and the
// launcher of the per-(row, chunk) dot kernel.
#pragma once

#include "xenc_common.h"

namespace xenc {

// Rank variant for C <= 64 (one chunk per lane): the top-k is a rank count instead of k dependent
// wave arg-max rounds.  Lane l publishes the 64-bit key (order_key(logit_l) << 32) | ~l, logit =
// dot * route_temp as the reference ranks it: a larger key is a larger logit, or the same logit
// at a lower index.  Every lane then counts the keys above its own (LDS broadcast reads, one
// 64-bit compare per chunk, no branches): the ranks are a permutation of [0, C), and the lane of
// rank r < nsel is round r of the arg-max variant.  The softmax max is the rank-0 logit (the
// max over the kept lanes when dense); the exponentials go to LDS by position and are summed in
// position order.  LDS: dots[64] (read, then reused for the exponentials), keys[64] (8-byte
// aligned, in the taken / order scratch of at least 128 words).
__device__ __forceinline__ void select_topk_softmax_rank(float* dots, unsigned long long* keys, int C,
                                                         int top_k, int kk, float route_temp,
                                                         float* wrow, int* irow, float* selrow,
                                                         int lane) {
  const bool dense = top_k <= 0 || top_k >= C;
  const int nsel = min(dense ? C : top_k, kk);
  const float x = lane < C ? dots[lane] * route_temp : 0.f;
  const unsigned long long key =
      lane < C ? ((unsigned long long)order_key(x) << 32) | (unsigned)~lane : 0ull;
  const int C8 = (C + 7) & ~7;              // keys past C are 0: below every real key
  if (lane < C8) keys[lane] = key;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  int rank = 0;
  for (int j = 0; j < C8; j += 8) {
    unsigned long long kj[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) kj[u] = keys[j + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) rank += kj[u] > key ? 1 : 0;
  }
  const int pos = dense ? lane : rank;
  const bool has = lane < C && pos < nsel;
  // Softmax max: the top logit (position 0) under top-k; the max over the kept lanes when dense.
  float* es = dots;                          // the kept exponentials by position, 0 up to nsel8
  if (!dense && pos == 0 && lane < C) es[0] = x;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const float lmax = dense ? wave_max(has ? x : -INFINITY) : es[0];
  const float e = has ? expf(x - lmax) : 0.f;
  const int nsel8 = (nsel + 7) & ~7;
  __builtin_amdgcn_wave_barrier();           // every lane has read es[0]
  if (has) es[pos] = e;
  if (lane >= nsel && lane < nsel8) es[lane] = 0.f;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float sum = 0.f;                           // position order
  for (int r = 0; r < nsel8; r += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = es[r + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) sum += v[u];
  }
  const float inv = 1.f / sum;
  if (has) {
    const float wr = e * inv;
    irow[pos] = lane;
    selrow[pos] = wr;
    wrow[lane] = wr;
  }
  for (int r = nsel + lane; r < kk; r += kWave) {
    irow[r] = -1;
    selrow[r] = 0.f;
  }
}

// One q . S dot by one wave (d <= 256 * CB4, d % 4 == 0, both rows 16-byte aligned): lane-owned
// float4 columns accumulated in block order, then the wave sum.  Every routing dot of the decode
// paths is this function, so they agree bit for bit.
template <int CB4>
__device__ __forceinline__ float route_dot_wave(const float* __restrict__ qrow,
                                                const float* __restrict__ srow, int d, int lane) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  float4 qv[CB4];
  f32x4 sv[CB4];
#pragma unroll
  for (int cb = 0; cb < CB4; ++cb) {
    const int i = (cb * kWave + lane) * 4;
    qv[cb] = i < d ? *reinterpret_cast<const float4*>(qrow + i) : make_float4(0.f, 0.f, 0.f, 0.f);
    // Default cache policy: the nontemporal hint measured slower here (5.97 against 5.27 us on
    // 64 rows x 2177 chunks, 9.62 against 7.03 us on 64 rows over 8 libraries of 64 chunks).
    sv[cb] = *reinterpret_cast<const f32x4*>(srow + min(i, d - 4));
  }
  float a = 0.f;
#pragma unroll
  for (int cb = 0; cb < CB4; ++cb) {
    a = fmaf(qv[cb].x, sv[cb].x, a);
    a = fmaf(qv[cb].y, sv[cb].y, a);
    a = fmaf(qv[cb].z, sv[cb].z, a);
    a = fmaf(qv[cb].w, sv[cb].w, a);
  }
  return wave_sum(a);
}

// Two dots of one query row, q . s_a and q . s_b, with q loaded once and both summary rows in
// flight together; each is summed exactly as route_dot_wave sums it (bit-identical results).
template <int CB4>
__device__ __forceinline__ float2 route_dot2_wave(const float* __restrict__ qrow, const float* __restrict__ sa,
                                                  const float* __restrict__ sb, int d, int lane) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  float4 qv[CB4];
  f32x4 va[CB4], vb[CB4];
#pragma unroll
  for (int cb = 0; cb < CB4; ++cb) {
    const int i = (cb * kWave + lane) * 4;
    qv[cb] = i < d ? *reinterpret_cast<const float4*>(qrow + i) : make_float4(0.f, 0.f, 0.f, 0.f);
    va[cb] = *reinterpret_cast<const f32x4*>(sa + min(i, d - 4));
    vb[cb] = *reinterpret_cast<const f32x4*>(sb + min(i, d - 4));
  }
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int cb = 0; cb < CB4; ++cb) {
    a = fmaf(qv[cb].x, va[cb].x, a);
    a = fmaf(qv[cb].y, va[cb].y, a);
    a = fmaf(qv[cb].z, va[cb].z, a);
    a = fmaf(qv[cb].w, va[cb].w, a);
    b = fmaf(qv[cb].x, vb[cb].x, b);
    b = fmaf(qv[cb].y, vb[cb].y, b);
    b = fmaf(qv[cb].z, vb[cb].z, b);
    b = fmaf(qv[cb].w, vb[cb].w, b);
  }
  return make_float2(wave_sum(a), wave_sum(b));
}

// q . S dots of every (row, chunk) pair into w_dense [M, ldw] (one wave per dot; route.hip).
int launch_route_dots(const float* q, long long ldq, int M, int d, const float* S, const int* chunk_ptr,
                      const int* q_group, int G, float* w_dense, int ldw, hipStream_t st);

// Top-k + softmax of M rows whose dots are in w_dense [M, ldw], row m over the chunks of library
// q_group[m] (route_rows_select_kernel; route.hip).  Returns XENC_EINVAL when a row's LDS would
// not fit.
int launch_route_select(int M, const int* chunk_ptr, const int* q_group, int G, int top_k,
                        float route_temp, float* w_dense, int ldw, int* idx, float* w_sel, int kk,
                        hipStream_t st);

}  // namespace xenc
