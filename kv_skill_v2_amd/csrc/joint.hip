// Op B: the serving-side decode read of a document operator joined with the request's own rows
// (xenc/d23_read_kernels.py:31-47 is the math, :134-160 the calling contract).
//
// For query row n and kv head h with its G query heads (GQA):
//   keys / values = [ operator pool rows 0 .. op_len[n]-1 (block table op_bt[n])
//                   ; own pool rows      0 .. own_len[n]-1 (block table own_bt[n]) ]
//   out[n, h*G + g] = softmax_l(scale * <q[n, h*G+g], K_l>) . V_l       (one softmax over both)
// Pools are [num_blocks, block_size, Hkv, D] (fp16 or bf16, D contiguous).
//
// One launch.  Workgroup (n, h, split s) streams keys [s*chunk, (s+1)*chunk) of the joined range
// (the last split also takes any keys past nsplit*chunk, so none is ever dropped) and keeps an
// online max / sum / accumulator per query head in the log2 domain.  A key row of D elements is
// read by a group of D/8 lanes (16-byte loads; groups padded to a power of two), so a wave reads
// 64/TPR keys per step; 4 keys per lane group are in flight (block-table lookups first, then the
// K / V loads) and enter the online softmax as one block; score sums run on DPP and the
// permlane swaps.  Lane groups merge by shuffles, the 4 waves through LDS, and wave 0 writes the
// split's partial.  Launches of 256 or more workgroups merge the partials of each (n, h) in a
// second kernel (joint_merge_kernel); in smaller ones the last split of (n, h) to arrive
// (release / acquire on a per-(n, h) counter) merges them and re-arms the counter, so the
// workspace is zeroed once and stays valid across calls and graph replays.  Either way the
// partials are merged in split order by the same code: results are deterministic and equal.
#include <algorithm>

#include "xenc_common.h"

namespace xenc {
namespace {

constexpr int kJointThreads = 256;
constexpr int kJointWaves = kJointThreads / kWave;
constexpr int kKeysInFlight = 4;
constexpr int kMergeStates = 1024;   // split states (S x G) the last split stages in LDS

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// 8 consecutive elements -> fp32.
template <typename T> __device__ __forceinline__ void to_f32(const u32x4_t& v, float (&f)[8]);
template <> __device__ __forceinline__ void to_f32<_Float16>(const u32x4_t& v, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned w = v[i];
    f[2 * i] = (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xffffu));
    f[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
  }
}
template <> __device__ __forceinline__ void to_f32<__bf16>(const u32x4_t& v, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned w = v[i];
    f[2 * i] = __uint_as_float(w << 16);
    f[2 * i + 1] = __uint_as_float(w & 0xffff0000u);
  }
}

struct JointArgs {
  const void* q; long long s_qn, s_qh;
  const void* op_k; const void* op_v; long long op_sb, op_ss, op_sh; int op_bs;
  const int* op_bt; long long op_bts; const int* op_len;
  const void* own_k; const void* own_v; long long own_sb, own_ss, own_sh; int own_bs;
  const int* own_bt; long long own_bts; const int* own_len;
  int hkv, d, tpr, nsplit, chunk;
  int op_shift, own_shift;   // log2 of the block sizes when they are powers of two, else -1
  float scale_log2;
  float* out; long long s_on, s_oh;
  int* counters; float2* part_ml; float* part_acc;   // [N*Hkv], [N*Hkv][S][G], [N*Hkv][S][G][D]
  int two_pass;   // merge in joint_merge_kernel instead of the last split of each (row, kv head)
};

// Launches of at least this many workgroups merge in a second kernel; smaller ones (few rows,
// latency-bound) merge in the last split of each (row, kv head) and save the launch.
constexpr long long kJointTwoPassBlocks = 256;

// Sum over each aligned group of tpr lanes (tpr a power of two <= 64, uniform over the launch)
// for all N values at once: each step of group_sum that the group width needs is one uniform
// branch over the whole array.
template <int N>
__device__ __forceinline__ void group_sums_rt(float (&v)[N], int tpr) {
  if (tpr >= 2) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_f<0xB1>(v[i]);
  }
  if (tpr >= 4) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_f<0x4E>(v[i]);
  }
  if (tpr >= 8) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_f<0x141>(v[i]);
  }
  if (tpr >= 16) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += dpp_f<0x140>(v[i]);
  }
  if (tpr >= 32) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const unsigned u = __float_as_uint(v[i]);
      const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
      v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
  }
  if (tpr >= 64) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const unsigned u = __float_as_uint(v[i]);
      const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
      v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
  }
}

// Online-softmax merge of state (mo, lo, ao) into (m, l, a); all in the log2 domain.
__device__ __forceinline__ void lse_merge(float& m, float& l, float (&a)[8], float mo, float lo,
                                          const float (&ao)[8]) {
  const float mn = fmaxf(m, mo);
  const float c0 = mn == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mn);
  const float c1 = mn == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mo - mn);
  l = l * c0 + lo * c1;
#pragma unroll
  for (int e = 0; e < 8; ++e) a[e] = a[e] * c0 + ao[e] * c1;
  m = mn;
}

// After the split's partial is written: publish it (release, then a per-(row, kv head) arrival
// count); the last split of (n, h) to arrive acquires and merges the S partials in split order,
// writes the output rows and re-arms the counter.
template <int G>
__device__ __forceinline__ void merge_partials(const JointArgs& A, int nh, int S, int n, int h);

template <int G>
__device__ __forceinline__ void publish_and_merge(const JointArgs& A, int nh, int S, int n, int h,
                                                  bool& is_last_s) {
  if (A.two_pass) return;   // joint_merge_kernel merges after the launch
  __syncthreads();
  if (threadIdx.x == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const int prev = __hip_atomic_fetch_add(&A.counters[nh], 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    const bool last = prev == S - 1;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    is_last_s = last;
  }
  __syncthreads();
  if (!is_last_s) return;
  merge_partials<G>(A, nh, S, n, h);
  if (threadIdx.x == 0) atomicExch(&A.counters[nh], 0);
}

// The S partials of (row n, kv head h) merged in split order into the output rows.
template <int G>
__device__ __forceinline__ void merge_partials(const JointArgs& A, int nh, int S, int n, int h) {
  const long long p0 = (long long)nh * S;
  if (S * G <= kMergeStates) {
    // Split states to LDS; per head the max M, then per (split, head) the factor 2^(m - M) (0 for
    // an empty split) and the denominator in split order; then every output sums its S partial
    // accumulators in split order, 8 loads in flight.
    __shared__ float2 sml[kMergeStates];
    __shared__ float coef[kMergeStates];
    __shared__ float den[8];
    for (int i = threadIdx.x; i < S * G; i += kJointThreads) sml[i] = A.part_ml[p0 * G + i];
    __syncthreads();
    if (threadIdx.x < G) {
      const int g = threadIdx.x;
      float M = -INFINITY;
      for (int j = 0; j < S; ++j)
        if (sml[j * G + g].y > 0.f) M = fmaxf(M, sml[j * G + g].x);
      float dsum = 0.f;
      for (int j = 0; j < S; ++j) {
        const float2 ml = sml[j * G + g];
        const float c = ml.y > 0.f ? __builtin_amdgcn_exp2f(ml.x - M) : 0.f;
        coef[j * G + g] = c;
        dsum += c * ml.y;
      }
      den[g] = dsum;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < G * A.d; i += kJointThreads) {
      const int g = i / A.d, dd = i % A.d;
      const float* src = A.part_acc + (p0 * G + g) * A.d + dd;   // split j at src[j * G * d]
      const long long js = (long long)G * A.d;
      float num = 0.f;
      int j = 0;
      for (; j + 8 <= S; j += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = src[(j + u) * js];
#pragma unroll
        for (int u = 0; u < 8; ++u) num += coef[(j + u) * G + g] * v[u];
      }
      for (; j < S; ++j) num += coef[j * G + g] * src[j * js];
      A.out[n * A.s_on + (long long)(h * G + g) * A.s_oh + dd] = den[g] > 0.f ? num / den[g] : 0.f;
    }
  } else {
    for (int i = threadIdx.x; i < G * A.d; i += kJointThreads) {
      const int g = i / A.d, dd = i % A.d;
      float M = -INFINITY;
      for (int j = 0; j < S; ++j) {
        const float2 ml = A.part_ml[(p0 + j) * G + g];
        if (ml.y > 0.f) M = fmaxf(M, ml.x);
      }
      float num = 0.f, dsum = 0.f;
      for (int j = 0; j < S; ++j) {
        const float2 ml = A.part_ml[(p0 + j) * G + g];
        if (ml.y > 0.f) {
          const float c = __builtin_amdgcn_exp2f(ml.x - M);
          dsum += c * ml.y;
          num += c * A.part_acc[((p0 + j) * G + g) * A.d + dd];
        }
      }
      A.out[n * A.s_on + (long long)(h * G + g) * A.s_oh + dd] = dsum > 0.f ? num / dsum : 0.f;
    }
  }
}

// Second pass of a large launch: one workgroup per (row, kv head).  The stream order publishes the
// partials, so no workgroup of the read pays a release / acquire and no merge runs on its tail
// (32 rows x 16,448 keys, 1,024 workgroups: 0.413 -> 0.380 ms per call).
template <int G>
__global__ __launch_bounds__(kJointThreads) void joint_merge_kernel(JointArgs A) {
  const int nh = blockIdx.x;
  merge_partials<G>(A, nh, A.nsplit, nh / A.hkv, nh % A.hkv);
}

// TPR: the lanes per key row when fixed at compile time (16 for head dim 128, 32 for 256), so the
// score sums are straight-line code; 0 takes it from the arguments.
template <typename T, int G, int TPR>
__global__ __launch_bounds__(kJointThreads) void joint_read_kernel(JointArgs A) {
  __shared__ float lds_acc[2][G][512];
  __shared__ float lds_ml[2][G][2];
  __shared__ bool is_last_s;

  // Launch order (row, split, kv head): the kv heads of one key range run side by side, so a pool
  // row's heads (adjacent in memory) are read together.
  const int S = A.nsplit;
  const int h = blockIdx.x % A.hkv;
  const int s = (blockIdx.x / A.hkv) % S;
  const int n = blockIdx.x / (A.hkv * S);
  const int nh = n * A.hkv + h;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int tpr = TPR > 0 ? TPR : A.tpr;   // lanes per key row (power of two, >= D/8)
  const int lr = lane & (tpr - 1);
  const int grp = lane / tpr;
  const int groups = kWave / tpr;        // keys per wave step
  const int dim0 = lr * 8;
  const bool active = dim0 < A.d;
  const int dimc = min(dim0, A.d - 8);   // padding lanes (q = 0) read a valid column

  // q of the G heads, pre-scaled into the log2 domain.
  float qf[G][8];
  {
    const T* qb = static_cast<const T*>(A.q) + n * A.s_qn + (long long)h * G * A.s_qh;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      u32x4_t v = active ? *reinterpret_cast<const u32x4_t*>(qb + g * A.s_qh + dim0) : (u32x4_t){};
      to_f32<T>(v, qf[g]);
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[g][e] *= A.scale_log2;
    }
  }
  const int lo = A.op_len[n];
  const int L = lo + A.own_len[n];
  const int k0 = s * A.chunk;
  const int k1 = s == S - 1 ? L : min(L, k0 + A.chunk);

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }
  const T* opk = static_cast<const T*>(A.op_k);
  const T* opv = static_cast<const T*>(A.op_v);
  const T* owk = static_cast<const T*>(A.own_k);
  const T* owv = static_cast<const T*>(A.own_v);
  const int* opbt = A.op_bt + n * A.op_bts;
  const int* owbt = A.own_bt + n * A.own_bts;

  const int step = kJointWaves * groups;              // keys per workgroup step
  const int stride = step * kKeysInFlight;
  // Block and row of the kKeysInFlight keys base, base + step, ... (block 0 for keys past k1, which
  // load nothing).  The next iteration's lookups are issued while this one's keys are in flight,
  // so the table loads are off the critical path.
  // Keys past k1 are clamped to k1 - 1 (a valid key of a non-empty split): every table and row
  // load is in bounds and unconditional, and those keys are masked out of the softmax.
  const bool pow2 = A.op_shift >= 0 && A.own_shift >= 0;   // uniform: block sizes 2^k take shifts
  auto lookup = [&](int base, int (&blk)[kKeysInFlight], int (&row)[kKeysInFlight]) {
#pragma unroll
    for (int u = 0; u < kKeysInFlight; ++u) {
      const int key = min(base + u * step, k1 - 1);
      const bool ow = key >= lo;
      const int kk = ow ? key - lo : key;
      int bi;
      if (pow2) {
        const int sh = ow ? A.own_shift : A.op_shift;
        bi = kk >> sh;
        row[u] = kk & ((1 << sh) - 1);
      } else {
        const int bs = ow ? A.own_bs : A.op_bs;
        bi = kk / bs;
        row[u] = kk - bi * bs;
      }
      const int* tb = ow ? owbt : opbt;
      blk[u] = tb[bi];
    }
  };
  // Strides are below 2^31 (checked on the host): the block base is one 64-bit multiply-add and
  // the offset inside the block 32-bit.
  const unsigned op_sb = (unsigned)A.op_sb, op_ss = (unsigned)A.op_ss, own_sb = (unsigned)A.own_sb,
                 own_ss = (unsigned)A.own_ss;
  const unsigned op_h = (unsigned)(h * A.op_sh), own_h = (unsigned)(h * A.own_sh);
  int blk[kKeysInFlight], brow[kKeysInFlight];
  const int first = k0 + wv * groups + grp;
  if (k0 < k1) lookup(first, blk, brow);   // workgroup-uniform: an empty split loads nothing
  for (int base = first; base < k1; base += stride) {
    long long offk[kKeysInFlight];
    bool own[kKeysInFlight], live[kKeysInFlight];
#pragma unroll
    for (int u = 0; u < kKeysInFlight; ++u) {
      const int key = base + u * step;
      live[u] = key < k1;
      own[u] = min(key, k1 - 1) >= lo;
      offk[u] = own[u] ? (unsigned long long)(unsigned)blk[u] * own_sb + (brow[u] * own_ss + own_h)
                       : (unsigned long long)(unsigned)blk[u] * op_sb + (brow[u] * op_ss + op_h);
    }
    u32x4_t kv[kKeysInFlight], vv[kKeysInFlight];
#pragma unroll
    for (int u = 0; u < kKeysInFlight; ++u) {
      const T* kp = (own[u] ? owk : opk) + offk[u] + dimc;
      const T* vp = (own[u] ? owv : opv) + offk[u] + dimc;
      kv[u] = *reinterpret_cast<const u32x4_t*>(kp);
      vv[u] = *reinterpret_cast<const u32x4_t*>(vp);
    }
    lookup(base + stride, blk, brow);
    // Scores of the lane group's kKeysInFlight keys, then one online-softmax update per head for
    // the block (one max update and one accumulator rescale), then the values.
    float sc[kKeysInFlight][G];
    float flat[kKeysInFlight * G];
#pragma unroll
    for (int u = 0; u < kKeysInFlight; ++u) {
      float kf[8];
      to_f32<T>(kv[u], kf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float x = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) x = fmaf(qf[g][e], kf[e], x);
        flat[u * G + g] = x;
      }
    }
    group_sums_rt(flat, tpr);
#pragma unroll
    for (int u = 0; u < kKeysInFlight; ++u)
#pragma unroll
      for (int g = 0; g < G; ++g) sc[u][g] = flat[u * G + g];
    float c[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mn = m[g];
#pragma unroll
      for (int u = 0; u < kKeysInFlight; ++u) mn = live[u] ? fmaxf(mn, sc[u][g]) : mn;
      c[g] = mn == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[g] - mn);   // 0 before the first key
      float ls = l[g] * c[g];
#pragma unroll
      for (int u = 0; u < kKeysInFlight; ++u) {
        sc[u][g] = live[u] ? __builtin_amdgcn_exp2f(sc[u][g] - mn) : 0.f;
        ls += sc[u][g];
      }
      l[g] = ls;
      m[g] = mn;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] *= c[g];
    }
#pragma unroll
    for (int u = 0; u < kKeysInFlight; ++u) {
      float vf[8];
      to_f32<T>(vv[u], vf);
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(sc[u][g], vf[e], acc[g][e]);
    }
  }

  // Lane groups of a wave hold the same dims for different keys: butterfly merge.
  for (int o = tpr; o < kWave; o <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float ao[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) ao[e] = shfl_xor(acc[g][e], o);
      const float mo = shfl_xor(m[g], o), lo2 = shfl_xor(l[g], o);
      lse_merge(m[g], l[g], acc[g], mo, lo2, ao);
    }
  }
  // Waves 2,3 -> 0,1, then 1 -> 0, through LDS (group 0 lanes carry the wave's state).
  for (int half = kJointWaves / 2; half >= 1; half >>= 1) {
    if (wv >= half && wv < 2 * half && grp == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (active) {
#pragma unroll
          for (int e = 0; e < 8; ++e) lds_acc[wv - half][g][dim0 + e] = acc[g][e];
        }
        if (lr == 0) {
          lds_ml[wv - half][g][0] = m[g];
          lds_ml[wv - half][g][1] = l[g];
        }
      }
    }
    __syncthreads();
    if (wv < half && grp == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float ao[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) ao[e] = active ? lds_acc[wv][g][dim0 + e] : 0.f;
        lse_merge(m[g], l[g], acc[g], lds_ml[wv][g][0], lds_ml[wv][g][1], ao);
      }
    }
    __syncthreads();
  }
  // Wave 0 (group 0) writes the split's partial.
  const long long part = (long long)nh * S + s;
  if (wv == 0 && grp == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (lr == 0) A.part_ml[part * G + g] = make_float2(m[g], l[g]);
      if (active) {
        float* dst = A.part_acc + (part * G + g) * A.d + dim0;
#pragma unroll
        for (int e = 0; e < 8; ++e) dst[e] = acc[g][e];
      }
    }
  }
  publish_and_merge<G>(A, nh, S, n, h, is_last_s);
}

__global__ void joint_zero_kernel(int* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct JointLayout {
  size_t counters, ml, acc, total;
};

// [counters: max_n*Hkv ints | (m, l) per (n, h, split, head) | acc per (n, h, split, head, dim)].
// The counter region depends only on the capacity max_n, so counters zeroed once stay in place
// whatever row counts later calls use.
JointLayout joint_layout(int max_n, int N, int hkv, int nsplit, int g, int d) {
  JointLayout L;
  const size_t units = (size_t)N * hkv;
  L.counters = 0;
  L.ml = align256((size_t)max_n * hkv * sizeof(int));
  L.acc = align256(L.ml + units * nsplit * g * sizeof(float2));
  L.total = align256(L.acc + units * nsplit * g * (size_t)d * sizeof(float));
  return L;
}

// MFMA form for head dims 128 and 256 (fp16 / bf16 pools, G <= 8).  Same split, launch order,
// partial layout and merge as joint_read_kernel; inside a split, wave w takes the 16-key tiles
// w, w + 4, ... of its range.
//   Loads (WIDE: launches of 256 or more workgroups): the tile's K rows are read whole (each load
//   instruction covers 512 / D key rows, D / 8 lanes a row, 16 bytes a lane), as the V rows are,
//   and every pool load is nontemporal (each row is read once); a stream-only probe of this shape
//   read the same bytes at 6.8-6.9 TB/s this way against 6.1 TB/s with K straight in the MFMA
//   layout (16 rows x 64 bytes per instruction).  Smaller, latency-bound launches load K in the
//   MFMA layout directly, with the default policy (the clamped re-reads of a split's last key then
//   hit in cache): the LDS round trips of the whole-row form cost them more than the loads gain.
//   Scores: one v_mfma_f32_16x16x32 per 32 dims, A = the tile's 16 key rows (lane l: key l % 16,
//   dims 8 (l / 16) .. +8 of each 32-dim block; WIDE: read back from the wave's LDS rows), B = q^T (lane
//   l: query head l % 16 of the kv head, zero past G), so lane l receives the scores of keys
//   4 (l / 16) + i, head l % 16.
//   Softmax: per head in the log2 domain over the tile (max and sum across the four lanes of a
//   head by the permlane swaps), one accumulator rescale per tile.
//   Values: lane l owns dims l * D/64 .. +D/64 of every head; the tile's weights and V row
//   addresses pass through this wave's LDS slot, and each key is D/64 FMAs per head.
// Keys past the split end are clamped to its last key (all loads in bounds) and get weight 0.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

template <bool NT, typename V>
__device__ __forceinline__ V load_pool(const void* p) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const V*>(p));
  return *reinterpret_cast<const V*>(p);
}

template <typename T>
__device__ __forceinline__ f32x4_t mfma16x16x32(const u32x4_t& a, const u32x4_t& b, f32x4_t c) {
  if constexpr (__is_same(T, __bf16))
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ float half_to_f32(unsigned bits16) {
  if constexpr (__is_same(T, __bf16))
    return __uint_as_float(bits16 << 16);
  else
    return (float)__builtin_bit_cast(_Float16, (unsigned short)bits16);
}

constexpr int kTileKeys = 16;

template <typename T, int G, int D, bool WIDE>
__global__ __launch_bounds__(kJointThreads) void joint_read_mfma_kernel(JointArgs A) {
  constexpr int KB = D / 32;    // 32-dim blocks of a key row; also K load instructions per tile
  constexpr int DPL = D / 64;   // value dims per lane
  constexpr int LPR = D / 8;    // lanes per key row in the whole-row K loads
  constexpr int KPI = 64 / LPR; // key rows per K load instruction
  constexpr int KLD = D / 2 + 8;  // words per staged K row: 8 mod 64, so neither the row stores
                                  // (LPR lanes a row) nor the MFMA-layout reads conflict
  static_assert(D == 128 || D == 256, "the MFMA form covers head dims 128 and 256");
  static_assert(KB * KPI == kTileKeys, "one tile's K rows in KB load instructions");
  __shared__ float lds_acc[2][G][D];
  __shared__ __align__(16) unsigned lds_k[WIDE ? kJointWaves : 1][kTileKeys][WIDE ? KLD : 4];   // tile K rows
  __shared__ float lds_ml[2][G][2];
  __shared__ __align__(16) float lds_p[kJointWaves][kTileKeys][8];   // tile weights [key][head]
  __shared__ long long lds_v[kJointWaves][kTileKeys];   // tile V rows: offset, own pool as ~offset
  __shared__ float lds_c[kJointWaves][8];                            // tile rescale per head
  __shared__ bool is_last_s;

  const int S = A.nsplit;
  const int h = blockIdx.x % A.hkv;
  const int s = (blockIdx.x / A.hkv) % S;
  const int n = blockIdx.x / (A.hkv * S);
  const int nh = n * A.hkv + h;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int l16 = lane & 15, lq = lane >> 4;

  // q^T fragments of the G heads (raw 16-bit values; heads past G are zero).
  u32x4_t qf[KB];
  {
    const T* qrow = static_cast<const T*>(A.q) + n * A.s_qn + (long long)(h * G + min(l16, G - 1)) * A.s_qh;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(qrow + kb * 32 + 8 * lq);
      qf[kb] = l16 < G ? v : (u32x4_t){};
    }
  }
  const int lo = A.op_len[n];
  const int L = lo + A.own_len[n];
  const int k0 = s * A.chunk;
  const int k1 = s == S - 1 ? L : min(L, k0 + A.chunk);

  const T* opk = static_cast<const T*>(A.op_k);
  const T* opv = static_cast<const T*>(A.op_v);
  const T* owk = static_cast<const T*>(A.own_k);
  const T* owv = static_cast<const T*>(A.own_v);
  const int* opbt = A.op_bt + n * A.op_bts;
  const int* owbt = A.own_bt + n * A.own_bts;
  const bool pow2 = A.op_shift >= 0 && A.own_shift >= 0;
  const unsigned op_sb = (unsigned)A.op_sb, op_ss = (unsigned)A.op_ss, own_sb = (unsigned)A.own_sb,
                 own_ss = (unsigned)A.own_ss;
  const unsigned op_h = (unsigned)(h * A.op_sh), own_h = (unsigned)(h * A.own_sh);
  // V rows are passed between lanes as element offsets (the own pool's as ~offset) and loaded
  // through the kernel-argument pool pointers: global loads, not flat ones, whose completion would
  // also hold up every LDS wait behind them.

  float m = -INFINITY, l = 0.f;   // softmax state of head l16 (the same in its four lanes)
  float acc[G][DPL];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[g][j] = 0.f;

  // Block and row of key tb + l16 (clamped to k1 - 1), pool chosen by the key.  Only the table
  // load is issued here; the row offset is formed when the tile is issued, so no wait for it
  // holds up the loads already in flight.
  auto locate = [&](int tb, int& blk, int& row, bool& ow) {
    const int key = min(tb + l16, k1 - 1);
    ow = key >= lo;
    const int kk = ow ? key - lo : key;
    int bi;
    if (pow2) {
      const int sh = ow ? A.own_shift : A.op_shift;
      bi = kk >> sh;
      row = kk & ((1 << sh) - 1);
    } else {
      const int bs = ow ? A.own_bs : A.op_bs;
      bi = kk / bs;
      row = kk - bi * bs;
    }
    blk = (ow ? owbt : opbt)[bi];
  };

  constexpr int kWaveStride = kTileKeys * kJointWaves;
  // Issue the K fragments and V slices of the tile whose row offset this lane holds (key
  // tb + l16): the V row addresses go through this wave's LDS slot to every lane.
  auto issue = [&](int blk, int row, bool ow, u32x4_t (&kf)[KB], unsigned (&vraw)[kTileKeys][DPL / 2]) {
    const unsigned long long off = ow ? (unsigned long long)(unsigned)blk * own_sb + (row * own_ss + own_h)
                                      : (unsigned long long)(unsigned)blk * op_sb + (row * op_ss + op_h);
    if constexpr (!WIDE) {   // this lane's key row, straight in the MFMA layout
      const T* kp = (ow ? owk : opk) + off;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) kf[kb] = *reinterpret_cast<const u32x4_t*>(kp + kb * 32 + 8 * lq);
    }
    if (lq == 0) lds_v[wv][l16] = ow ? ~(long long)off : (long long)off;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    if constexpr (WIDE) {
      // K rows whole: instruction j covers keys KPI j .. KPI j + KPI - 1, lane l key KPI j + l / LPR,
      // dims 8 (l % LPR) .. +8 (staged to the MFMA layout when the tile is consumed).
#pragma unroll
      for (int j = 0; j < KB; ++j) {
        const long long ko = lds_v[wv][j * KPI + lane / LPR];
        kf[j] = load_pool<true, u32x4_t>((ko < 0 ? owk + ~ko : opk + ko) + (lane % LPR) * 8);
      }
    }
#pragma unroll
    for (int k = 0; k < kTileKeys; ++k) {
      const long long vo = lds_v[wv][k];
      const T* vr = (vo < 0 ? owv + ~vo : opv + vo) + lane * DPL;
      if constexpr (DPL == 4) {
        const u32x2_t v2 = load_pool<WIDE, u32x2_t>(vr);
        vraw[k][0] = v2[0];
        vraw[k][1] = v2[1];
      } else {
        vraw[k][0] = load_pool<WIDE, unsigned>(vr);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();   // the slot is rewritten by the next issue
  };
  // Scores, softmax and values of tile tb from its loaded fragments.
  auto consume = [&](int tb, const u32x4_t (&kf)[KB], const unsigned (&vraw)[kTileKeys][DPL / 2]) {
    // WIDE: the tile's K rows through this wave's LDS rows, stored as loaded and read back in the
    // MFMA layout (lane l: row l % 16, dims kb * 32 + 8 (l / 16) .. +8).
    u32x4_t ka[KB];
    if constexpr (WIDE) {
#pragma unroll
      for (int j = 0; j < KB; ++j)
        *reinterpret_cast<u32x4_t*>(&lds_k[wv][j * KPI + lane / LPR][(lane % LPR) * 4]) = kf[j];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) ka[kb] = *reinterpret_cast<const u32x4_t*>(&lds_k[wv][l16][kb * 16 + 4 * lq]);
    } else {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) ka[kb] = kf[kb];
    }
    f32x4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) sacc = mfma16x16x32<T>(ka[kb], qf[kb], sacc);
    float sv[4];
    bool ok[4];
    float mt = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ok[i] = tb + 4 * lq + i < k1;
      sv[i] = sacc[i] * A.scale_log2;
      mt = ok[i] ? fmaxf(mt, sv[i]) : mt;
    }
    mt = fmaxf(mt, swap_partner<16>(mt, (lane & 16) != 0));
    mt = fmaxf(mt, swap_partner<32>(mt, (lane & 32) != 0));
    const float mn = fmaxf(m, mt);   // key tb < k1 is in every tile: mt is finite
    const float c = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mn);
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sv[i] = ok[i] ? __builtin_amdgcn_exp2f(sv[i] - mn) : 0.f;
      ps += sv[i];
    }
    ps += swap_partner<16>(ps, (lane & 16) != 0);
    ps += swap_partner<32>(ps, (lane & 32) != 0);
    l = l * c + ps;
    m = mn;
    if (l16 < G) {
#pragma unroll
      for (int i = 0; i < 4; ++i) lds_p[wv][4 * lq + i][l16] = sv[i];
      if (lq == 0) lds_c[wv][l16] = c;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float cg = lds_c[wv][g];
#pragma unroll
      for (int j = 0; j < DPL; ++j) acc[g][j] *= cg;
    }
#pragma unroll
    for (int k = 0; k < kTileKeys; ++k) {
      float pk[8];
      const float4 p0 = *reinterpret_cast<const float4*>(&lds_p[wv][k][0]);
      pk[0] = p0.x; pk[1] = p0.y; pk[2] = p0.z; pk[3] = p0.w;
      if constexpr (G > 4) {
        const float4 p1 = *reinterpret_cast<const float4*>(&lds_p[wv][k][4]);
        pk[4] = p1.x; pk[5] = p1.y; pk[6] = p1.z; pk[7] = p1.w;
      }
      float vf[DPL];
#pragma unroll
      for (int j = 0; j < DPL; ++j) vf[j] = half_to_f32<T>(j & 1 ? vraw[k][j / 2] >> 16 : vraw[k][j / 2] & 0xffffu);
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[g][j] = fmaf(pk[g], vf[j], acc[g][j]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();   // the weight slot is rewritten by the next tile
  };

  // Steady state per tile t: the table lookup of t + 2 strides, the K / V loads of t + 1, then t is
  // consumed.  Every lookup and load is issued unconditionally (keys past the split clamp to its
  // last key, so the extra loads re-read rows already in cache); only the consumes stop at the
  // wave's last tile.  Loads complete in order, so each wait covers just the tile it needs.
  u32x4_t kfa[KB], kfb[KB];
  unsigned vra[kTileKeys][DPL / 2], vrb[kTileKeys][DPL / 2];
  int blka, blkb, rowa, rowb;
  bool owa, owb;
  const int t0 = k0 + kTileKeys * wv;
  if (t0 < k1) {   // wave-uniform
    locate(t0, blka, rowa, owa);
    locate(t0 + kWaveStride, blkb, rowb, owb);
    issue(blka, rowa, owa, kfa, vra);
    for (int tb = t0;; tb += 2 * kWaveStride) {
      locate(tb + 2 * kWaveStride, blka, rowa, owa);
      issue(blkb, rowb, owb, kfb, vrb);
      consume(tb, kfa, vra);
      if (tb + kWaveStride >= k1) break;
      locate(tb + 3 * kWaveStride, blkb, rowb, owb);
      issue(blka, rowa, owa, kfa, vra);
      consume(tb + kWaveStride, kfb, vrb);
      if (tb + 2 * kWaveStride >= k1) break;
    }
  }

  // Per-head state as wave-uniform values (lane g holds head g).
  float Mg[G], Lg[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    Mg[g] = readlane(m, g);
    Lg[g] = readlane(l, g);
  }
  // Waves 2,3 -> 0,1, then 1 -> 0, through LDS.
  for (int half = kJointWaves / 2; half >= 1; half >>= 1) {
    if (wv >= half && wv < 2 * half) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int j = 0; j < DPL; ++j) lds_acc[wv - half][g][lane * DPL + j] = acc[g][j];
        if (lane == 0) {
          lds_ml[wv - half][g][0] = Mg[g];
          lds_ml[wv - half][g][1] = Lg[g];
        }
      }
    }
    __syncthreads();
    if (wv < half) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float m2 = lds_ml[wv][g][0], l2 = lds_ml[wv][g][1];
        const float M = fmaxf(Mg[g], m2);
        const float a = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(Mg[g] - M);
        const float b = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m2 - M);
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[g][j] = acc[g][j] * a + lds_acc[wv][g][lane * DPL + j] * b;
        Lg[g] = Lg[g] * a + l2 * b;
        Mg[g] = M;
      }
    }
    __syncthreads();
  }
  const long long part = (long long)nh * S + s;
  if (wv == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (lane == 0) A.part_ml[part * G + g] = make_float2(Mg[g], Lg[g]);
      float* dst = A.part_acc + (part * G + g) * A.d + lane * DPL;
#pragma unroll
      for (int j = 0; j < DPL; ++j) dst[j] = acc[g][j];
    }
  }
  publish_and_merge<G>(A, nh, S, n, h, is_last_s);
}

template <typename T, int G>
void launch_joint_g(dim3 grid, hipStream_t st, const JointArgs& a) {
  // Whole-row nontemporal pool loads in the two-pass (large) launches only.
  if (a.d == 256 && a.two_pass)
    hipLaunchKernelGGL((joint_read_mfma_kernel<T, G, 256, true>), grid, dim3(kJointThreads), 0, st, a);
  else if (a.d == 256)
    hipLaunchKernelGGL((joint_read_mfma_kernel<T, G, 256, false>), grid, dim3(kJointThreads), 0, st, a);
  else if (a.d == 128 && a.two_pass)
    hipLaunchKernelGGL((joint_read_mfma_kernel<T, G, 128, true>), grid, dim3(kJointThreads), 0, st, a);
  else if (a.d == 128)
    hipLaunchKernelGGL((joint_read_mfma_kernel<T, G, 128, false>), grid, dim3(kJointThreads), 0, st, a);
  else if (a.tpr == 32)
    hipLaunchKernelGGL((joint_read_kernel<T, G, 32>), grid, dim3(kJointThreads), 0, st, a);
  else if (a.tpr == 16)
    hipLaunchKernelGGL((joint_read_kernel<T, G, 16>), grid, dim3(kJointThreads), 0, st, a);
  else
    hipLaunchKernelGGL((joint_read_kernel<T, G, 0>), grid, dim3(kJointThreads), 0, st, a);
}

template <typename T, int G>
void launch_joint_both(dim3 grid, hipStream_t st, const JointArgs& a) {
  launch_joint_g<T, G>(grid, st, a);
  if (a.two_pass)
    hipLaunchKernelGGL((joint_merge_kernel<G>), dim3(grid.x / a.nsplit), dim3(kJointThreads), 0, st, a);
}

template <typename T>
int launch_joint(int G, dim3 grid, hipStream_t st, const JointArgs& a) {
  switch (G) {
    case 1: launch_joint_both<T, 1>(grid, st, a); break;
    case 2: launch_joint_both<T, 2>(grid, st, a); break;
    case 3: launch_joint_both<T, 3>(grid, st, a); break;
    case 4: launch_joint_both<T, 4>(grid, st, a); break;
    case 5: launch_joint_both<T, 5>(grid, st, a); break;
    case 6: launch_joint_both<T, 6>(grid, st, a); break;
    case 7: launch_joint_both<T, 7>(grid, st, a); break;
    case 8: launch_joint_both<T, 8>(grid, st, a); break;
    default: return XENC_EINVAL;
  }
  return check_launch();
}

}  // namespace
}  // namespace xenc

using namespace xenc;

extern "C" size_t xenc_joint_workspace_bytes(int max_n, int hkv, int nsplit, int g, int d) {
  if (max_n < 0 || hkv <= 0 || nsplit <= 0 || g <= 0 || d <= 0) return 0;
  return joint_layout(max_n, max_n, hkv, nsplit, g, d).total;
}

extern "C" int xenc_joint_workspace_init(void* workspace, size_t workspace_bytes, int max_n, int hkv,
                                         void* stream) {
  if (max_n < 0 || hkv <= 0) return XENC_EINVAL;
  const long long n = (long long)max_n * hkv;
  if (n == 0) return XENC_OK;
  if (!workspace) return XENC_ENULL;
  if (workspace_bytes < (size_t)n * sizeof(int)) return XENC_EWORKSPACE;
  const int blocks = (int)std::min<long long>((n + 255) / 256, 1024);
  hipLaunchKernelGGL(joint_zero_kernel, dim3(blocks), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<int*>(workspace), (int)n);
  return check_launch();
}

extern "C" int xenc_paged_decode_joint(
    int dtype, int N, int hq, int hkv, int d,
    const void* q, long long s_qn, long long s_qh,
    const void* op_k, const void* op_v, long long op_sb, long long op_ss, long long op_sh, int op_bs,
    const int* op_bt, long long op_bt_stride, const int* op_len,
    const void* own_k, const void* own_v, long long own_sb, long long own_ss, long long own_sh,
    int own_bs, const int* own_bt, long long own_bt_stride, const int* own_len,
    float scale, int nsplit, int chunk, float* out, long long s_on, long long s_oh,
    void* workspace, size_t workspace_bytes, int max_n, void* stream) {
  if (dtype != 0 && dtype != 1) return XENC_EINVAL;
  if (N < 0 || hq <= 0 || hkv <= 0 || hq % hkv != 0) return XENC_EINVAL;
  if (N > max_n) return XENC_EWORKSPACE;
  const int G = hq / hkv;
  if (G > 8 || d <= 0 || d % 8 != 0 || d > 512 || G * d > 4096) return XENC_EINVAL;
  if (nsplit <= 0 || nsplit > 4096 || chunk <= 0 || op_bs <= 0 || own_bs <= 0) return XENC_EINVAL;
  if (s_qh < d || s_qn < (long long)hq * s_qh || s_oh < d || s_on < (long long)hq * s_oh) return XENC_EINVAL;
  for (long long st : {s_qn, s_qh, op_sb, op_ss, op_sh, own_sb, own_ss, own_sh})
    if (st % 8 != 0 || st < 0) return XENC_EALIGN;
  // One pool block (and a kv head's offset inside it) stays below 2^31 elements.
  for (long long st : {op_sb, own_sb, (long long)op_bs * op_ss, (long long)own_bs * own_ss,
                       (long long)hkv * op_sh, (long long)hkv * own_sh})
    if (st >= (1LL << 31)) return XENC_EINVAL;
  if (N == 0) return XENC_OK;
  if (!q || !op_k || !op_v || !op_bt || !op_len || !own_k || !own_v || !own_bt || !own_len ||
      !out || !workspace)
    return XENC_ENULL;
  for (const void* p : {q, op_k, op_v, own_k, own_v, (const void*)out, (const void*)workspace})
    if (!aligned16(p)) return XENC_EALIGN;
  const JointLayout lay = joint_layout(max_n, N, hkv, nsplit, G, d);
  if (workspace_bytes < lay.total) return XENC_EWORKSPACE;
  int tpr = 1;
  while (tpr * 8 < d) tpr <<= 1;
  auto shift_of = [](int bs) {
    if (bs & (bs - 1)) return -1;
    int sh = 0;
    while ((1 << sh) < bs) ++sh;
    return sh;
  };
  char* ws = static_cast<char*>(workspace);
  JointArgs a{q, s_qn, s_qh, op_k, op_v, op_sb, op_ss, op_sh, op_bs, op_bt, op_bt_stride, op_len,
              own_k, own_v, own_sb, own_ss, own_sh, own_bs, own_bt, own_bt_stride, own_len,
              hkv, d, tpr, nsplit, chunk, shift_of(op_bs), shift_of(own_bs), scale * kLog2e, out, s_on, s_oh,
              reinterpret_cast<int*>(ws + lay.counters), reinterpret_cast<float2*>(ws + lay.ml),
              reinterpret_cast<float*>(ws + lay.acc), 0};
  const long long blocks = (long long)N * hkv * nsplit;
  if (blocks > 0x7fffffffLL) return XENC_EINVAL;
  a.two_pass = blocks >= kJointTwoPassBlocks ? 1 : 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  return dtype == 0 ? launch_joint<_Float16>(G, dim3((unsigned)blocks), st, a)
                    : launch_joint<__bf16>(G, dim3((unsigned)blocks), st, a);
}
