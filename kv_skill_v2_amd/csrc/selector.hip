// LayerSelector on the device (xenc/selector.py:59-110) and the gate * gain row scale of the
// epilogue (xenc/injector.py:59-69):
//
//   selector_weights_kernel  per row b of logits z [B, n]: keep the top k (descending, ties to the
//                            lower index), w = softmax over the kept logits, 0 elsewhere;
//                            dense w [B, n] and the kept (index, weight) pairs in rank order
//   selector_apply_kernel    out[b] = sum_{j<k} w[b,j] * alpha * delta[b*k+j] / (rel + 1e-6),
//                            rel = |delta[b*k+j]| / (|h[b]| + 1e-6), alpha = exp(*log_alpha): the
//                            matched-norm rescale and weighting of LayerSelector.apply, summed
//                            over the k selected layers of a token (k = 1: apply itself);
//                            selector_apply_regs_kernel, the same for k <= 2 with the rows held
//                            in registers (one pass of loads, one workgroup sum for all norms)
//   gate_scale_kernel        scale[m] = gain_scale * exp(log_gain[p]) *
//                            sigmoid(<hn[t], gate_w> + gate_b[p]), t = row_token[m],
//                            p = row_pos[m]: the per-row factor of delta = scale * B(r)
//   multi_depth_prepare_kernel  selector_weights and gate_scale for the multi-depth decode step
//                            in one launch: per token the selector top-k, the kept depths' query
//                            rows gathered and their row scales
// Every sum runs in a fixed order (deterministic).
#include <climits>

#include "route_select.h"
#include "xenc_common.h"

namespace xenc {
namespace {

constexpr int kSelMaxN = 256;   // candidates per row (4 per lane)

// Top-k + softmax of one row of logits zr (n candidates) by one wave: dense weights into wr
// (n entries), the kept (index, weight) pairs in rank order into idx / w_sel.
__device__ __forceinline__ void select_weights_row(const float* __restrict__ zr, int n, int k, int lane,
                                                   float* __restrict__ wr, int* __restrict__ idx,
                                                   float* __restrict__ w_sel) {
  // Candidate c carries the 64-bit key (order_key(z_c) << 32) | ~c: a larger key is a larger
  // logit (NaN above +inf, as topk ranks it) or the same logit at a lower index.  Every real
  // candidate's key is nonzero, taken and padding entries are 0, so each of the k <= n rounds
  // picks an untaken candidate in [0, n), whatever the logits hold.
  float v[4];
  unsigned long long key[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int c = lane + u * kWave;
    v[u] = c < n ? zr[c] : -INFINITY;
    key[u] = c < n ? ((unsigned long long)order_key(v[u]) << 32) | (unsigned)~c : 0ull;
  }
  float kept_v = -INFINITY;   // lane j < k ends with the j-th kept value and index
  int kept_i = 0;
  if (n <= kWave) {
    // One candidate per lane: its rank is the number of larger keys (the keys are distinct),
    // counted over the n lanes by readlane; the candidate of rank r then goes to lane r.  The
    // same selection as the rounds below, without their cross-lane shuffles.
    const unsigned klo = (unsigned)key[0], khi = (unsigned)(key[0] >> 32);
    int rank = 0;
    for (int c = 0; c < n; ++c) {
      const unsigned long long kc =
          ((unsigned long long)(unsigned)__builtin_amdgcn_readlane((int)khi, c) << 32) |
          (unsigned)__builtin_amdgcn_readlane((int)klo, c);
      rank += kc > key[0] ? 1 : 0;
    }
    for (int r = 0; r < k; ++r) {
      const unsigned long long hit = __ballot(lane < n && rank == r);
      // Exactly one lane has rank r < k <= n.
      const int c = __builtin_amdgcn_readfirstlane((int)__builtin_ctzll(hit));
      const float vc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[0]), c));
      if (lane == r) {
        kept_v = vc;
        kept_i = c;
      }
    }
  }
  for (int r = 0; n > kWave && r < k; ++r) {
    unsigned long long best = key[0];
#pragma unroll
    for (int u = 1; u < 4; ++u) best = key[u] > best ? key[u] : best;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const unsigned lo = shfl_xor((int)(unsigned)best, o);
      const unsigned hi = shfl_xor((int)(unsigned)(best >> 32), o);
      const unsigned long long other = ((unsigned long long)hi << 32) | lo;
      best = other > best ? other : best;
    }
    const int bi = min(max((int)~(unsigned)best, 0), n - 1);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (lane + u * kWave == bi) key[u] = 0ull;
    if (lane == r) {
      kept_v = zr[bi];
      kept_i = bi;
    }
  }
  // Softmax over the kept values (lanes 0..k-1).
  const float m = wave_max(lane < k ? kept_v : -INFINITY);
  const float e = lane < k ? __expf(kept_v - m) : 0.f;
  const float s = wave_sum(e);
  const float wk = e / s;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int c = lane + u * kWave;
    if (c < n) wr[c] = 0.f;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  if (lane < k) {
    wr[kept_i] = wk;
    idx[lane] = kept_i;
    w_sel[lane] = wk;
  }
}

// One wave per row.
__global__ __launch_bounds__(256) void selector_weights_kernel(
    const float* __restrict__ z, long long ldz, int B, int n, int k, float* __restrict__ w,
    long long ldw, int* __restrict__ idx, float* __restrict__ w_sel, long long lds) {
  const int lane = threadIdx.x & (kWave - 1);
  const int b = blockIdx.x * 4 + threadIdx.x / kWave;
  if (b >= B) return;  // wave-uniform
  select_weights_row(z + (long long)b * ldz, n, k, lane, w + (long long)b * ldw, idx + (long long)b * lds,
                     w_sel + (long long)b * lds);
}

// Workgroup sum of one float per thread (kRowThreads threads), fixed order.
constexpr int kRowThreads = 256;
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Sum over e < d of f(a[e], b[e]) by the workgroup: 16-byte loads when vec4 (d, both rows 16-byte
// aligned), else scalar.  Each thread accumulates its elements in order; then a fixed-order
// workgroup sum.
template <typename F>
__device__ __forceinline__ float row_dot(const float* a, const float* b, int d, bool vec4, float* red, F f) {
  float acc = 0.f;
  if (vec4) {
    const int d4 = d / 4;
#pragma unroll 4
    for (int i = threadIdx.x; i < d4; i += kRowThreads) {
      const f32x4 x = reinterpret_cast<const f32x4*>(a)[i];
      const f32x4 y = reinterpret_cast<const f32x4*>(b)[i];
      acc = f(x[0], y[0], acc);
      acc = f(x[1], y[1], acc);
      acc = f(x[2], y[2], acc);
      acc = f(x[3], y[3], acc);
    }
  } else {
#pragma unroll 4
    for (int e = threadIdx.x; e < d; e += kRowThreads) acc = f(a[e], b[e], acc);
  }
  return block_sum(acc, red);
}

struct Fma {
  __device__ float operator()(float x, float y, float acc) const { return fmaf(x, y, acc); }
};

// selector_apply_kernel for 16-byte rows of d <= 4 * kRowThreads * kApplyPer and K <= 2 kept
// layers: the thread's pieces of h and of the K update rows load together and stay in registers,
// the K + 1 norms are summed in one fixed-order workgroup pass, and the output comes from the
// registers.  Every sum runs in the order of row_dot / block_sum and of the general kernel's
// output loop, so the result is bit-identical to it.
constexpr int kApplyPer = 8;
template <int K>
__global__ __launch_bounds__(kRowThreads) void selector_apply_regs_kernel(
    int d, const float* __restrict__ delta, long long ldd, const float* __restrict__ h, long long ldh,
    const float* __restrict__ w_row, const float* __restrict__ log_alpha, float* __restrict__ out,
    long long ldo) {
  __shared__ float red[K + 1][kRowThreads / kWave];
  const int b = blockIdx.x;
  const int d4 = d / 4;
  const f32x4* rows[K + 1];
  rows[0] = reinterpret_cast<const f32x4*>(h + (long long)b * ldh);
#pragma unroll
  for (int j = 0; j < K; ++j) rows[j + 1] = reinterpret_cast<const f32x4*>(delta + ((long long)b * K + j) * ldd);
  f32x4 x[K + 1][kApplyPer];
#pragma unroll
  for (int u = 0; u < kApplyPer; ++u) {
    const int i = min((int)threadIdx.x + u * kRowThreads, d4 - 1);   // clamped: unconditional loads
#pragma unroll
    for (int j = 0; j <= K; ++j) x[j][u] = rows[j][i];
  }
  float ss[K + 1];
#pragma unroll
  for (int j = 0; j <= K; ++j) {
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < kApplyPer; ++u)
      if ((int)threadIdx.x + u * kRowThreads < d4) {
        acc = fmaf(x[j][u][0], x[j][u][0], acc);
        acc = fmaf(x[j][u][1], x[j][u][1], acc);
        acc = fmaf(x[j][u][2], x[j][u][2], acc);
        acc = fmaf(x[j][u][3], x[j][u][3], acc);
      }
    ss[j] = wave_sum(acc);
  }
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j <= K; ++j) red[j][wv] = ss[j];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j <= K; ++j) ss[j] = (red[j][0] + red[j][1]) + (red[j][2] + red[j][3]);
  const float hnorm = sqrtf(ss[0]);
  const float alpha = __expf(*log_alpha);
  float coef[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const float rel = sqrtf(ss[j + 1]) / (hnorm + 1e-6f);
    coef[j] = w_row[(long long)b * K + j] * alpha / (rel + 1e-6f);
  }
  f32x4* o = reinterpret_cast<f32x4*>(out + (long long)b * ldo);
#pragma unroll
  for (int u = 0; u < kApplyPer; ++u) {
    const int i = (int)threadIdx.x + u * kRowThreads;
    if (i < d4) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < K; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = fmaf(coef[j], x[j + 1][u][e], acc[e]);
      o[i] = acc;
    }
  }
}

// One workgroup per output row b.
__global__ __launch_bounds__(kRowThreads) void selector_apply_kernel(
    int k, int d, const float* __restrict__ delta, long long ldd, const float* __restrict__ h,
    long long ldh, const float* __restrict__ w_row, const float* __restrict__ log_alpha,
    float* __restrict__ out, long long ldo, int vec4) {
  __shared__ float red[kRowThreads / kWave];
  __shared__ float coef_s[64];
  const int b = blockIdx.x;
  const float* hb = h + (long long)b * ldh;
  const float hnorm = sqrtf(row_dot(hb, hb, d, vec4, red, Fma()));
  const float alpha = __expf(*log_alpha);
  for (int j = 0; j < k; ++j) {
    const float* dr = delta + ((long long)b * k + j) * ldd;
    const float dnorm = sqrtf(row_dot(dr, dr, d, vec4, red, Fma()));
    if (threadIdx.x == 0) {
      const float rel = dnorm / (hnorm + 1e-6f);
      coef_s[j] = w_row[(long long)b * k + j] * alpha / (rel + 1e-6f);
    }
  }
  __syncthreads();
  float* o = out + (long long)b * ldo;
  const float* d0 = delta + (long long)b * k * ldd;
  if (vec4) {
    for (int i = threadIdx.x; i < d / 4; i += kRowThreads) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int j = 0; j < k; ++j) {
        const f32x4 x = reinterpret_cast<const f32x4*>(d0 + (long long)j * ldd)[i];
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[u] = fmaf(coef_s[j], x[u], acc[u]);
      }
      reinterpret_cast<f32x4*>(o)[i] = acc;
    }
  } else {
    for (int e = threadIdx.x; e < d; e += kRowThreads) {
      float acc = 0.f;
      for (int j = 0; j < k; ++j) acc = fmaf(coef_s[j], d0[(long long)j * ldd + e], acc);
      o[e] = acc;
    }
  }
}

// One workgroup per query row m.
__global__ __launch_bounds__(kRowThreads) void gate_scale_kernel(
    [[maybe_unused]] int M, int d, const float* __restrict__ hn, long long ldh, const int* __restrict__ row_token,
    const int* __restrict__ row_pos, int n_pos, const float* __restrict__ gate_w,
    const float* __restrict__ gate_b, const float* __restrict__ log_gain, float gain_scale,
    float* __restrict__ scale, int vec4) {
  __shared__ float red[kRowThreads / kWave];
  const int m = blockIdx.x;
  const int t = row_token ? row_token[m] : m;
  const int p = min(max(row_pos ? row_pos[m] : 0, 0), n_pos - 1);
  const float s = row_dot(hn + (long long)t * ldh, gate_w, d, vec4, red, Fma());
  if (threadIdx.x == 0) {
    const float g = 1.f / (1.f + __expf(-(s + gate_b[p])));
    scale[m] = gain_scale * __expf(log_gain[p]) * g;
  }
}

// The multi-depth step's per-token work in one launch, one workgroup per token b: the selector
// top-k of z[b] (select_weights_row, wave 0), then the query row of each kept depth copied from
// q_all into q_rows[b*k + j], and the row scale of each kept depth from the token's gate dot
// (row_dot, the gate_scale_kernel sum).  Each output is bit-identical to the separate kernel's.
struct PrepareArgs {
  const float* z; long long ldz; int n, k;
  const float* q_all; long long q_depth_stride, q_token_stride; int d;
  const float* hn; long long ldh; int d_r;
  const float *gate_w, *gate_b, *log_gain; float gain_scale;
  float* w; long long ldw; int* idx; float* w_sel; long long lds;
  float* q_rows; long long ldr; float* scale; int vec4_q, vec4_h;
};

// Token b's work by the first kRowThreads threads of a workgroup (red: kRowThreads / kWave
// floats, kept: 64 ints of LDS).
__device__ __forceinline__ void prepare_token(int b, const PrepareArgs& a, float* red, int* kept) {
  const float* __restrict__ z = a.z;
  const long long ldz = a.ldz;
  const int n = a.n, k = a.k, d = a.d, d_r = a.d_r, vec4_q = a.vec4_q, vec4_h = a.vec4_h;
  const float* __restrict__ q_all = a.q_all;
  const long long q_depth_stride = a.q_depth_stride, q_token_stride = a.q_token_stride;
  const float* __restrict__ hn = a.hn;
  const long long ldh = a.ldh;
  const float* __restrict__ gate_w = a.gate_w;
  const float* __restrict__ gate_b = a.gate_b;
  const float* __restrict__ log_gain = a.log_gain;
  const float gain_scale = a.gain_scale;
  float* __restrict__ w = a.w;
  const long long ldw = a.ldw, lds = a.lds, ldr = a.ldr;
  int* __restrict__ idx = a.idx;
  float* __restrict__ w_sel = a.w_sel;
  float* __restrict__ q_rows = a.q_rows;
  float* __restrict__ scale = a.scale;
  const int lane = threadIdx.x & (kWave - 1);
  const float* hrow = hn + (long long)b * ldh;
  // 16-byte rows of d_r <= 4 * kRowThreads * kApplyPer: this thread's pieces of the gate dot load
  // before the selection, so that their latency overlaps it, and are summed afterwards in
  // row_dot's order (bit-identical to gate_scale_kernel's sum).
  const int d4 = d_r / 4;
  const bool pre = vec4_h && d4 <= kRowThreads * kApplyPer;
  f32x4 hx[kApplyPer], gx[kApplyPer];
  if (pre) {
#pragma unroll
    for (int u = 0; u < kApplyPer; ++u) {
      const int i = min((int)threadIdx.x + u * kRowThreads, d4 - 1);   // clamped: unconditional loads
      hx[u] = reinterpret_cast<const f32x4*>(hrow)[i];
      gx[u] = reinterpret_cast<const f32x4*>(gate_w)[i];
    }
  }
  if (threadIdx.x < kWave) {
    select_weights_row(z + (long long)b * ldz, n, k, lane, w + (long long)b * ldw, idx + (long long)b * lds,
                       w_sel + (long long)b * lds);
    if (lane < k) kept[lane] = idx[(long long)b * lds + lane];
  }
  // The gate dot does not depend on the selection; block_sum's barriers also publish kept[].
  float s;
  if (pre) {
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < kApplyPer; ++u)
      if ((int)threadIdx.x + u * kRowThreads < d4) {
        acc = fmaf(hx[u][0], gx[u][0], acc);
        acc = fmaf(hx[u][1], gx[u][1], acc);
        acc = fmaf(hx[u][2], gx[u][2], acc);
        acc = fmaf(hx[u][3], gx[u][3], acc);
      }
    s = block_sum(acc, red);
  } else {
    s = row_dot(hrow, gate_w, d_r, vec4_h, red, Fma());
  }
  // The kept depths' query rows, up to four rows' loads in flight before their stores.
  for (int j0 = 0; j0 < k; j0 += 4) {
    const float* src[4];
    float* dst[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = min(j0 + jj, k - 1);
      src[jj] = q_all + (long long)kept[j] * q_depth_stride + (long long)b * q_token_stride;
      dst[jj] = q_rows + ((long long)b * k + j) * ldr;
    }
    const int nj = min(4, k - j0);
    if (vec4_q) {
#pragma unroll 2
      for (int i = threadIdx.x; i < d / 4; i += kRowThreads) {
        f32x4 t[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) t[jj] = reinterpret_cast<const f32x4*>(src[jj])[i];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          if (jj < nj) reinterpret_cast<f32x4*>(dst[jj])[i] = t[jj];
      }
    } else {
      for (int e = threadIdx.x; e < d; e += kRowThreads) {
        float t[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) t[jj] = src[jj][e];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          if (jj < nj) dst[jj][e] = t[jj];
      }
    }
  }
  if (threadIdx.x < k) {
    const int p = kept[threadIdx.x];
    const float g = 1.f / (1.f + __expf(-(s + gate_b[p])));
    scale[(long long)b * k + threadIdx.x] = gain_scale * __expf(log_gain[p]) * g;
  }
}

__global__ __launch_bounds__(kRowThreads) void multi_depth_prepare_kernel(PrepareArgs a) {
  __shared__ float red[kRowThreads / kWave];
  __shared__ int kept[64];
  prepare_token(blockIdx.x, a, red, kept);
}

// The per-token work above and the routing dots of the step's rows in one launch.  Workgroup
// (b, 0) runs prepare_token(b); workgroup (b, 1 + j * ncb + cb) takes chunks 4cb .. 4cb + 3 of
// row b*k + j, one wave per chunk, with route_dot_wave (the dots of route_dots_kernel, bit for
// bit).  Its depth, the candidate of rank j in z[b], is ranked here from the same 64-bit keys
// as select_weights_row (n <= 64), so the dots do not wait for the selection's launch; the query
// row is read from q_all, of which q_rows[b*k + j] is a copy.
template <int CB4>
__global__ __launch_bounds__(kRowThreads) void multi_depth_prepare_dots_kernel(
    PrepareArgs a, int ncb, const float* __restrict__ S, const int* __restrict__ chunk_ptr, int G,
    float* __restrict__ dots, int ldd) {
  __shared__ float red[kRowThreads / kWave];
  __shared__ int kept[64];
  const int b = blockIdx.x;
  if (blockIdx.y == 0) {
    prepare_token(b, a, red, kept);
    return;
  }
  const int lane = threadIdx.x & (kWave - 1);
  const int j = (blockIdx.y - 1) / ncb;
  const int c = ((blockIdx.y - 1) % ncb) * (kRowThreads / kWave) + (int)(threadIdx.x / kWave);
  const float v = lane < a.n ? a.z[(long long)b * a.ldz + lane] : -INFINITY;
  const unsigned long long key =
      lane < a.n ? ((unsigned long long)order_key(v) << 32) | (unsigned)~lane : 0ull;
  const unsigned klo = (unsigned)key, khi = (unsigned)(key >> 32);
  int rank = 0;
  for (int i = 0; i < a.n; ++i) {
    const unsigned long long ki =
        ((unsigned long long)(unsigned)__builtin_amdgcn_readlane((int)khi, i) << 32) |
        (unsigned)__builtin_amdgcn_readlane((int)klo, i);
    rank += ki > key ? 1 : 0;
  }
  const unsigned long long hit = __ballot(lane < a.n && rank == j);   // one lane: j < k <= n
  const int depth = min(__builtin_amdgcn_readfirstlane((int)__builtin_ctzll(hit | (1ull << 63))), a.n - 1);
  const int g = min(max(depth, 0), G - 1);
  const int c0 = chunk_ptr[g];
  const int C = min(chunk_ptr[g + 1] - c0, ldd);
  if (c >= C) return;
  const float* qrow = a.q_all + (long long)depth * a.q_depth_stride + (long long)b * a.q_token_stride;
  const float x = route_dot_wave<CB4>(qrow, S + (long long)(c0 + c) * a.d, a.d, lane);
  if (lane == 0) dots[((long long)b * a.k + j) * ldd + c] = x;
}

}  // namespace
}  // namespace xenc

using namespace xenc;

extern "C" int xenc_selector_weights(const float* z, long long ldz, int B, int n, int k, float* w,
                                     long long ldw, int* idx, float* w_sel, long long ld_sel,
                                     void* stream) {
  if (B < 0 || n <= 0 || n > kSelMaxN || k <= 0 || k > n || k > kWave || ldz < n || ldw < n ||
      ld_sel < k)
    return XENC_EINVAL;
  if (B == 0) return XENC_OK;
  if (!z || !w || !idx || !w_sel) return XENC_ENULL;
  hipLaunchKernelGGL(selector_weights_kernel, dim3((B + 3) / 4), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), z, ldz, B, n, k, w, ldw, idx, w_sel, ld_sel);
  return check_launch();
}

extern "C" int xenc_selector_apply(int B, int k, int d, const float* delta, long long ldd,
                                   const float* h, long long ldh, const float* w_row,
                                   const float* log_alpha, float* out, long long ldo, void* stream) {
  if (B < 0 || k <= 0 || k > 64 || d <= 0 || ldd < d || ldh < d || ldo < d) return XENC_EINVAL;
  if (B == 0) return XENC_OK;
  if (!delta || !h || !w_row || !log_alpha || !out) return XENC_ENULL;
  const int vec4 = (d % 4 == 0 && ldd % 4 == 0 && ldh % 4 == 0 && ldo % 4 == 0 && aligned16(delta) &&
                    aligned16(h) && aligned16(out)) ? 1 : 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (vec4 && k <= 2 && d / 4 <= kRowThreads * kApplyPer) {
    if (k == 1)
      hipLaunchKernelGGL(selector_apply_regs_kernel<1>, dim3(B), dim3(kRowThreads), 0, st, d, delta, ldd, h, ldh,
                         w_row, log_alpha, out, ldo);
    else
      hipLaunchKernelGGL(selector_apply_regs_kernel<2>, dim3(B), dim3(kRowThreads), 0, st, d, delta, ldd, h, ldh,
                         w_row, log_alpha, out, ldo);
    return check_launch();
  }
  hipLaunchKernelGGL(selector_apply_kernel, dim3(B), dim3(kRowThreads), 0, st, k, d, delta, ldd, h, ldh, w_row,
                     log_alpha, out, ldo, vec4);
  return check_launch();
}

extern "C" int xenc_gate_scale(int M, int d, const float* hn, long long ldh, const int* row_token,
                               const int* row_pos, int n_pos, const float* gate_w, const float* gate_b,
                               const float* log_gain, float gain_scale, float* scale, void* stream) {
  if (M < 0 || d <= 0 || ldh < d || n_pos <= 0) return XENC_EINVAL;
  if (M == 0) return XENC_OK;
  if (!hn || !gate_w || !gate_b || !log_gain || !scale) return XENC_ENULL;
  const int vec4 = (d % 4 == 0 && ldh % 4 == 0 && aligned16(hn) && aligned16(gate_w)) ? 1 : 0;
  hipLaunchKernelGGL(gate_scale_kernel, dim3(M), dim3(kRowThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), M, d, hn, ldh, row_token, row_pos, n_pos,
                     gate_w, gate_b, log_gain, gain_scale, scale, vec4);
  return check_launch();
}

extern "C" int xenc_multi_depth_prepare(const float* z, long long ldz, int B, int n, int k,
                                        const float* q_all, long long q_depth_stride,
                                        long long q_token_stride, int d, const float* hn, long long ldh,
                                        int d_r, const float* gate_w, const float* gate_b,
                                        const float* log_gain, float gain_scale, float* w, long long ldw,
                                        int* idx, float* w_sel, long long ld_sel, float* q_rows,
                                        long long ldr, float* scale, void* stream) {
  if (B < 0 || n <= 0 || n > kSelMaxN || k <= 0 || k > n || k > kWave || ldz < n || ldw < n ||
      ld_sel < k || d <= 0 || d_r <= 0 || ldh < d_r || ldr < d)
    return XENC_EINVAL;
  if (q_depth_stride < 0 || q_token_stride < 0) return XENC_EINVAL;
  if (B == 0) return XENC_OK;
  if (!z || !q_all || !hn || !gate_w || !gate_b || !log_gain || !w || !idx || !w_sel || !q_rows || !scale)
    return XENC_ENULL;
  const int vec4_q = (d % 4 == 0 && q_depth_stride % 4 == 0 && q_token_stride % 4 == 0 && ldr % 4 == 0 &&
                      aligned16(q_all) && aligned16(q_rows)) ? 1 : 0;
  const int vec4_h = (d_r % 4 == 0 && ldh % 4 == 0 && aligned16(hn) && aligned16(gate_w)) ? 1 : 0;
  const PrepareArgs a{z, ldz, n, k, q_all, q_depth_stride, q_token_stride, d, hn, ldh, d_r, gate_w, gate_b,
                      log_gain, gain_scale, w, ldw, idx, w_sel, ld_sel, q_rows, ldr, scale, vec4_q, vec4_h};
  hipLaunchKernelGGL(multi_depth_prepare_kernel, dim3(B), dim3(kRowThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return check_launch();
}

extern "C" int xenc_multi_depth_prepare_route(
    const float* z, long long ldz, int B, int n, int k, const float* q_all, long long q_depth_stride,
    long long q_token_stride, int d, const float* hn, long long ldh, int d_r, const float* gate_w,
    const float* gate_b, const float* log_gain, float gain_scale, float* w, long long ldw, int* idx,
    float* w_sel, long long ld_sel, float* q_rows, long long ldr, float* scale, const float* S,
    const int* chunk_ptr, int G, int top_k, float route_temp, float* w_dense, long long ldwd,
    int* ridx, float* rw_sel, int kk, void* stream) {
  if (B < 0 || n <= 0 || n > kWave || k <= 0 || k > n || ldz < n || ldw < n || ld_sel < k || d <= 0 ||
      d_r <= 0 || ldh < d_r || ldr < d || G <= 0 || kk <= 0 || ldwd <= 0)
    return XENC_EINVAL;
  if (q_depth_stride < 0 || q_token_stride < 0) return XENC_EINVAL;
  if (d % 8 != 0 || d > 4096 || q_depth_stride % 4 != 0 || q_token_stride % 4 != 0) return XENC_EINVAL;
  if (ld_sel != k || (long long)B * k > INT_MAX / 2) return XENC_EINVAL;   // idx doubles as [B*k] libraries
  if (B == 0) return XENC_OK;
  if (!z || !q_all || !hn || !gate_w || !gate_b || !log_gain || !w || !idx || !w_sel || !q_rows || !scale ||
      !S || !chunk_ptr || !w_dense || !ridx || !rw_sel)
    return XENC_ENULL;
  if (!aligned16(q_all) || !aligned16(S)) return XENC_EALIGN;
  const int vec4_q = (ldr % 4 == 0 && aligned16(q_rows)) ? 1 : 0;
  const int vec4_h = (d_r % 4 == 0 && ldh % 4 == 0 && aligned16(hn) && aligned16(gate_w)) ? 1 : 0;
  const PrepareArgs a{z, ldz, n, k, q_all, q_depth_stride, q_token_stride, d, hn, ldh, d_r, gate_w, gate_b,
                      log_gain, gain_scale, w, ldw, idx, w_sel, ld_sel, q_rows, ldr, scale, vec4_q, vec4_h};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  constexpr int kChunksPerBlock = kRowThreads / kWave;
  const int ncb = (int)((ldwd + kChunksPerBlock - 1) / kChunksPerBlock);
  const dim3 grid(B, 1 + k * ncb);
  switch ((d + 255) / 256) {
#define XENC_PD(N)                                                                               \
  case N:                                                                                        \
    hipLaunchKernelGGL(multi_depth_prepare_dots_kernel<N>, grid, dim3(kRowThreads), 0, st, a, ncb, \
                       S, chunk_ptr, G, w_dense, (int)ldwd);                                     \
    break;
    XENC_PD(1) XENC_PD(2) XENC_PD(3) XENC_PD(4) XENC_PD(5) XENC_PD(6) XENC_PD(7) XENC_PD(8)
    XENC_PD(9) XENC_PD(10) XENC_PD(11) XENC_PD(12) XENC_PD(13) XENC_PD(14) XENC_PD(15) XENC_PD(16)
#undef XENC_PD
    default:
      return XENC_EINVAL;
  }
  // The rows' libraries are their depths, written by the workgroups (b, 0) above.
  return launch_route_select(B * k, chunk_ptr, idx, G, top_k, route_temp, w_dense, (int)ldwd, ridx, rw_sel,
                             kk, st);
}
