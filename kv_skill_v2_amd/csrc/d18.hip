// D18: a library of D documents' operators read by the reader's own query in one pass
// (lib_read, xenc/d18_library.py:34-96).  For reader row t, kv head h and its G query heads:
//
//   document d:  s_d = scale * qd[d] . K_d            (qd[d] rotated at N_d + P + t)
//                o_d = softmax([s_d ; s_own]) . [V_d ; V_own]
//                r_d = logsumexp(s_d[skip:]),  rmax_d = max(s_d[skip:])   (all of s_d if N_d <= skip)
//   own rows:    s_own = scale * qo . K_own[0 .. P + t]   (qo rotated at P + t; causal)
//   routing:     w = softmax_d(beta * r)  (top_k kept, ties to the lower index; or force / wfix)
//   output:      o = sum_d w_d o_d                     (before the gate and o_proj)
//
// Two launches.  d18_partials_kernel: one workgroup per (row, kv head, unit, key split), the
// units being the D documents and the own rows, each cut into S key ranges so that a few rows
// (decode) still spread over the GPU; it streams its keys once for all G query heads (GQA) with
// an online softmax in the log2 domain, and for a document also the max / sum of the keys past
// `skip`.  Scores of 16 keys x the G heads are one MFMA tile (fp16 operands split into hi + lo
// parts, fp32 accumulation); the value sums run on the VALU in fp32; the 4 waves merge through
// LDS in a fixed order.  d18_merge_kernel: one workgroup per
// (row, query head, 64 output dims) merges the splits, joins each document with the own rows
// (o_d), forms r, rmax and the routing weights, and sums w_d o_d.  Deterministic: every sum runs
// in a fixed order.
#include <algorithm>

#include "xenc_common.h"

namespace xenc {
namespace {

constexpr int kD18Threads = 256;                      // merge kernel
constexpr int kD18Waves = kD18Threads / kWave;
constexpr int kD18PartThreads = 256;                  // partials kernel (one wave per SIMD: 512 threads
                                                      // cap a wave at 256 registers and spill)
constexpr int kD18PartWaves = kD18PartThreads / kWave;
constexpr int kD18MaxG = 8;
constexpr int kD18MaxHd = 256;
constexpr int kD18MaxDocs = 64;
constexpr int kD18MaxSplits = 32;

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <typename T> struct D18Elem { static constexpr int EPL = 8; };   // 16-bit keys
template <> struct D18Elem<float> { static constexpr int EPL = 4; };

// 16 bytes of T (loaded as v) as EPL fp32 values.
template <typename T>
__device__ __forceinline__ void cvt_f32(const u32x4_t& v, float (&f)[D18Elem<T>::EPL]) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(v[i]);
  } else if constexpr (__is_same(T, __bf16)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(v[i] << 16);
      f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = (float)__builtin_bit_cast(_Float16, (unsigned short)(v[i] & 0xffffu));
      f[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (unsigned short)(v[i] >> 16));
    }
  }
}

// 16 bytes of T at p (16-byte aligned) as EPL fp32 values.
template <typename T>
__device__ __forceinline__ void load_f32(const T* p, float (&f)[D18Elem<T>::EPL]) {
  cvt_f32<T>(*reinterpret_cast<const u32x4_t*>(p), f);
}

// 2^(m - M) with m = -inf (an empty state) -> 0, also when M = -inf.
__device__ __forceinline__ float rescale(float m, float M) {
  return m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
}

typedef _Float16 d18_half8 __attribute__((ext_vector_type(8)));
constexpr int kD18Tile = 16;   // keys per score tile (the MFMA's 16 rows)

// LDS of one unit: per wave the probabilities of its current key tile [key][head] and the heads'
// rescale factors, then per wave and query head the state (m, l, mc, lc) and the accumulator.
constexpr int kD18KPad = 4;    // words of padding per staged row (conflict-free MFMA-layout reads)
constexpr int kD18KRow = kD18MaxHd + kD18KPad;   // words per staged key row (fp32 keys fill it)
// LDS of one unit: the query fragments (fp16 hi / lo rows of the 16 padded heads), per wave the
// raw key rows of its current tile and the tile's probabilities [key][head] with the heads'
// rescale factors, then per wave and query head the state (m, l, mc, lc) and the accumulator.
struct D18Lds {
  _Float16 qh[16][kD18MaxHd + 8], ql[16][kD18MaxHd + 8];
  unsigned k[kD18PartWaves][kD18Tile][kD18KRow];
  float p[kD18PartWaves][kD18Tile][16];
  float alpha[kD18PartWaves][16];
  float st[kD18PartWaves][kD18MaxG][4];
  float acc[kD18PartWaves][kD18MaxG][kD18MaxHd];
};

// x = hi + lo in fp16 with |x - hi - lo| <= 2^-22 |x| (for |x| in fp16's normal range).
__device__ __forceinline__ _Float16 f16_hi(float x) { return (_Float16)x; }
__device__ __forceinline__ _Float16 f16_lo(float x) { return (_Float16)(x - (float)(_Float16)x); }

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The G query rows q[g * HD ...] of a kv head, scaled to the log2 domain, into LDS as fp16
// hi + lo rows (padded heads 0): the B operand of the scores, read by every wave.  Ends with a
// workgroup barrier.
template <int HD>
__device__ __forceinline__ void stage_q(const float* __restrict__ q, int G, float scale_log2, D18Lds& lds) {
  for (int i = threadIdx.x; i < 16 * HD; i += kD18PartThreads) {
    const int g = i / HD, e = i % HD;
    const float x = g < G ? q[g * HD + e] * scale_log2 : 0.f;
    lds.qh[g][e] = f16_hi(x);
    lds.ql[g][e] = f16_lo(x);
  }
  __syncthreads();
}

// One key split (n keys, the first at index j_base of its unit; n <= 0: empty) for the G query
// heads of a kv head (staged by stage_q), hd = HD.  Wave wv takes the 16-key tiles wv, wv + 4, ...
// Scores on the matrix cores: S^T [16 keys x 16 heads] = K_tile . Q^T with
// v_mfma_f32_16x16x32_f16 (A = keys: lane holds key lane % 16 at dims 32 kb + 8 (lane / 16) + e;
// B = queries: head lane % 16, same dims), q split into fp16 hi + lo (two products; fp32 keys also
// split: three), so the scores keep fp32 accuracy.  Lane (k4 = lane / 16, head = lane % 16) then
// holds the scores of keys 4 k4 .. 4 k4 + 3 for its head: the online softmax per head is an
// in-lane step plus two xor shuffles, and the wave's (m, l) per head is uniform over the wave.
// The probabilities go through LDS to the value lanes: a V row of hd elements is read by
// TPR = HD / EPL lanes (16-byte loads), and acc[g][e] += p[key][g] v[e] in fp32.
// A tile's K and V rows load row-contiguous (16-byte loads, TPR lanes a row): the K rows go
// through LDS into the MFMA layout (loaded in that layout, every 16 lanes would touch 16 rows),
// the V rows stay in registers as loaded.  Rows past n re-read row n - 1 (their scores are
// masked).  (Loading the next tile during this one measured no faster: 18.1 against 17.4 us.)
// Keys at unit index >= skip_c (skip_c >= 0) also enter the content max / sum (mc, lc).  Writes
// ml_out[g] = (m, l, mc, lc) (log2 domain) and acc_out[g * HD + e] (unnormalised).
template <typename TK, int HD, int GP>
__device__ __forceinline__ void d18_unit(int G, const TK* __restrict__ K, const TK* __restrict__ V, long long s_n,
                                         int n, int j_base, int skip_c, float4* __restrict__ ml_out,
                                         float* __restrict__ acc_out, D18Lds& lds) {
  constexpr int EPL = D18Elem<TK>::EPL;
  constexpr int TPR = HD / EPL;              // lanes per row: a power of two <= 64
  constexpr int KPI = kWave / TPR;           // rows per wave load
  constexpr int NI = kD18Tile / KPI > 0 ? kD18Tile / KPI : 1;   // loads per tile (K or V)
  constexpr int KB = HD / 32;                // MFMA k steps
  constexpr int WPR = HD * (int)sizeof(TK) / 4;   // words per key row
  constexpr bool kF32 = sizeof(TK) == 4;
  static_assert(KPI <= kD18Tile, "a tile holds at least one wave load of rows");
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int hs = lane % 16, k4 = lane / 16;              // score layout
  const int grp = lane / TPR, e0 = (lane % TPR) * EPL;   // load / value layout
  const int w0 = e0 * (int)sizeof(TK) / 4;               // this lane's first word of a row
  float acc[GP][EPL];
#pragma unroll
  for (int g = 0; g < GP; ++g)
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
  float m = -INFINITY, l = 0.f, mc = -INFINITY, lc = 0.f;   // head hs
  // Content statistics of the split: none (own rows, or every key before skip_c), all (every key
  // at or past skip_c: then they equal (m, l) and are copied at the end), or per key (the split
  // that holds key skip_c).  Workgroup-uniform.
  const int cmode = skip_c < 0 || j_base + n <= skip_c ? 0 : j_base >= skip_c ? 1 : 2;
  auto load_rows = [&](const TK* base, int t0, u32x4_t (&r)[NI]) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
      r[i] = *reinterpret_cast<const u32x4_t*>(base + (long long)min(t0 + i * KPI + grp, n - 1) * s_n + e0);
  };
  for (int t0 = wv * kD18Tile; t0 < n; t0 += kD18PartWaves * kD18Tile) {
    {
      u32x4_t kr[NI], vr[NI];
      load_rows(K, t0, kr);
      load_rows(V, t0, vr);
      // The tile's K rows to LDS.
#pragma unroll
      for (int i = 0; i < NI; ++i) *reinterpret_cast<u32x4_t*>(&lds.k[wv][i * KPI + grp][w0]) = kr[i];
      wave_sync_lds();
      f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const d18_half8 qh = *reinterpret_cast<const d18_half8*>(&lds.qh[hs][32 * kb + 8 * k4]);
        const d18_half8 ql = *reinterpret_cast<const d18_half8*>(&lds.ql[hs][32 * kb + 8 * k4]);
        d18_half8 ka, kl;
        if constexpr (kF32) {
          const f32x4_t a = *reinterpret_cast<const f32x4_t*>(&lds.k[wv][hs][32 * kb + 8 * k4]);
          const f32x4_t b = *reinterpret_cast<const f32x4_t*>(&lds.k[wv][hs][32 * kb + 8 * k4 + 4]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            ka[e] = f16_hi(a[e]);
            kl[e] = f16_lo(a[e]);
            ka[4 + e] = f16_hi(b[e]);
            kl[4 + e] = f16_lo(b[e]);
          }
        } else {
          const u32x4_t kv = *reinterpret_cast<const u32x4_t*>(&lds.k[wv][hs][(32 * kb + 8 * k4) / 2]);
          float f[8];
          cvt_f32<TK>(kv, f);
#pragma unroll
          for (int e = 0; e < 8; ++e) ka[e] = (_Float16)f[e];
        }
        sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh, sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql, sc, 0, 0, 0);
        if constexpr (kF32) sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh, sc, 0, 0, 0);
      }
      // Online softmax of head hs over the tile's keys t0 + 4 k4 + r.
      bool ok[4];
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ok[r] = t0 + 4 * k4 + r < n;
        if (ok[r]) mx = fmaxf(mx, sc[r]);
      }
      mx = fmaxf(mx, shfl_xor(mx, 16));
      mx = fmaxf(mx, shfl_xor(mx, 32));
      const float mn = fmaxf(m, mx);
      const float a = rescale(m, mn);
      float pr[4], ps = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pr[r] = ok[r] ? __builtin_amdgcn_exp2f(sc[r] - mn) : 0.f;
        ps += pr[r];
      }
      ps += shfl_xor(ps, 16);
      ps += shfl_xor(ps, 32);
      l = l * a + ps;
      m = mn;
      if (cmode == 2) {
        float mcx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (ok[r] && j_base + t0 + 4 * k4 + r >= skip_c) mcx = fmaxf(mcx, sc[r]);
        mcx = fmaxf(mcx, shfl_xor(mcx, 16));
        mcx = fmaxf(mcx, shfl_xor(mcx, 32));
        const float mcn = fmaxf(mc, mcx);
        float cs = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (ok[r] && j_base + t0 + 4 * k4 + r >= skip_c) cs += __builtin_amdgcn_exp2f(sc[r] - mcn);
        cs += shfl_xor(cs, 16);
        cs += shfl_xor(cs, 32);
        lc = lc * rescale(mc, mcn) + cs;
        mc = mcn;
      }
      // Probabilities and rescale factors to the value lanes.
#pragma unroll
      for (int r = 0; r < 4; ++r) lds.p[wv][4 * k4 + r][hs] = pr[r];
      if (k4 == 0) lds.alpha[wv][hs] = a;
      wave_sync_lds();
#pragma unroll
      for (int g = 0; g < GP; ++g) {
        const float ag = lds.alpha[wv][g];
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] *= ag;
      }
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int key = i * KPI + grp;
        float vf[EPL];
        cvt_f32<TK>(vr[i], vf);
#pragma unroll
        for (int g = 0; g < GP; ++g) {
          const float pg = lds.p[wv][key][g];
#pragma unroll
          for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(pg, vf[e], acc[g][e]);
        }
      }
      wave_sync_lds();   // the next tile's keys and probabilities overwrite these
    }
  }
  if (cmode == 1) {
    mc = m;
    lc = l;
  }
  // Lane groups of the wave (same dims, different keys) share the wave's state: their sums add.
#pragma unroll
  for (int o = TPR; o < kWave; o <<= 1)
#pragma unroll
    for (int g = 0; g < GP; ++g)
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[g][e] += shfl_xor(acc[g][e], o);
  // The 4 waves through LDS, summed in wave order.
  if (grp == 0) {
#pragma unroll
    for (int g = 0; g < GP; ++g)
#pragma unroll
      for (int e = 0; e < EPL; ++e) lds.acc[wv][g][e0 + e] = acc[g][e];
  }
  if (lane < G) {
    lds.st[wv][lane][0] = m;
    lds.st[wv][lane][1] = l;
    lds.st[wv][lane][2] = mc;
    lds.st[wv][lane][3] = lc;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < G * HD; i += kD18PartThreads) {
    const int g = i / HD, e = i % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kD18PartWaves; ++w) M = fmaxf(M, lds.st[w][g][0]);
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kD18PartWaves; ++w) s += lds.acc[w][g][e] * rescale(lds.st[w][g][0], M);
    acc_out[i] = s;
  }
  if ((int)threadIdx.x < G) {
    const int g = threadIdx.x;
    float M = -INFINITY, Mc = -INFINITY;
#pragma unroll
    for (int w = 0; w < kD18PartWaves; ++w) {
      M = fmaxf(M, lds.st[w][g][0]);
      Mc = fmaxf(Mc, lds.st[w][g][2]);
    }
    float L = 0.f, Lc = 0.f;
#pragma unroll
    for (int w = 0; w < kD18PartWaves; ++w) {
      L += lds.st[w][g][1] * rescale(lds.st[w][g][0], M);
      Lc += lds.st[w][g][3] * rescale(lds.st[w][g][2], Mc);
    }
    ml_out[g] = make_float4(M, L, Mc, Lc);
  }
}

// Partials of split s of unit u of (row t, kv head h), blockIdx = (t * hkv + h, u * S + s); u < D
// a document (keys split into S ranges of ceil(N_d / S)), u = D the own rows (S ranges of
// ceil((P + T) / S), cut at row t's causal end P + t + 1).  Layout: part_ml [T][hkv][D + 1][S][G],
// part_acc [T][hkv][D + 1][S][G][hd].
template <typename TD, int HD, int GP>
__global__ __launch_bounds__(kD18PartThreads) void d18_partials_kernel(
    int hq, int hkv, int n_docs, int S, const float* __restrict__ qd, const float* __restrict__ qo,
    const TD* __restrict__ kd, const TD* __restrict__ vd, long long s_dh, long long s_dn,
    const int* __restrict__ doc_ptr, const float* __restrict__ ko, const float* __restrict__ vo,
    long long s_oh, long long s_on, int P, int T, float scale_log2, int skip,
    float4* __restrict__ part_ml, float* __restrict__ part_acc) {
  __shared__ D18Lds lds;
  const int th = blockIdx.x;
  const int t = th / hkv, h = th % hkv;
  const int u = blockIdx.y / S, sp = blockIdx.y % S;
  const int G = hq / hkv;
  const long long slot = (((long long)th * (n_docs + 1) + u) * S + sp) * G;
  // The query rows go to LDS first: they do not wait on the document offsets.
  stage_q<HD>(u < n_docs ? qd + (((long long)u * T + t) * hq + (long long)h * G) * HD
                         : qo + ((long long)t * hq + (long long)h * G) * HD,
              G, scale_log2, lds);
  if (u < n_docs) {
    const int n0 = doc_ptr[u], N = doc_ptr[u + 1] - n0;
    const int chunk = (N + S - 1) / S;
    const int lo = sp * chunk, n = min(N - lo, chunk);
    const long long off = (long long)h * s_dh + (long long)(n0 + lo) * s_dn;
    d18_unit<TD, HD, GP>(G, kd + off, vd + off, s_dn, n, lo, N > skip ? skip : 0, part_ml + slot,
                         part_acc + slot * HD, lds);
  } else {
    const int chunk = (P + T + S - 1) / S;
    const int lo = sp * chunk, n = min(P + t + 1 - lo, chunk);
    const long long off = (long long)h * s_oh + (long long)lo * s_on;
    d18_unit<float, HD, GP>(G, ko + off, vo + off, s_on, n, lo, -1, part_ml + slot, part_acc + slot * HD, lds);
  }
}

// One workgroup per (row t, kv head h, query head g) and block of 64 output dims:
// blockIdx.x = (t * hkv + h) * G + g, blockIdx.y = dim block.  The S splits of every unit are
// merged first (in split order): their rescale factors and the unit states go to LDS.  Wave 0
// forms the routing weights (one lane per document; block 0 writes w, r, rmax).  Then wave v
// merges the split accumulators of units v, v + 4, ... for the block's dims (lane = dim, all S
// loads of two units in flight) into LDS, and wave 0 sums o[e] = sum_d w_d o_d[e], o_d the join
// of document d and the own rows.
// w, r, rmax: [hkv][G][T][D] (the reference's [Hkv, G, T, D]); out: [T][hq][hd].
constexpr int kD18MergeDims = kWave;

__global__ __launch_bounds__(kD18Threads) void d18_merge_kernel(
    int T, int hq, int hkv, int hd, int n_docs, int S, const float4* __restrict__ part_ml,
    const float* __restrict__ part_acc, float beta, int top_k, int force, const float* __restrict__ wfix,
    float* __restrict__ out, float* __restrict__ w_out, float* __restrict__ r_out, float* __restrict__ rmax_out) {
  __shared__ float wl[kD18MaxDocs];
  __shared__ float4 ust[kD18MaxDocs + 1];                       // per unit: (M, L, Mc, Lc) over splits
  __shared__ float fac[(kD18MaxDocs + 1) * kD18MaxSplits];      // 2^(m_split - M_unit)
  __shared__ float4 sst[(kD18MaxDocs + 1) * kD18MaxSplits];     // the split states
  __shared__ float ua[kD18MaxDocs + 1][kD18MergeDims];          // per unit: the merged accumulator
  const int G = hq / hkv, U = n_docs + 1;
  const int g = blockIdx.x % G, th = blockIdx.x / G;
  const int t = th / hkv, h = th % hkv;
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  // slot of (unit u, split s): ((th * U + u) * S + s) * G + g
  auto slot = [&](int u, int sp) { return (((long long)th * U + u) * S + sp) * G + g; };
  // Split states to LDS (one load per thread), then per unit the max / sums in split order.
  for (int i = threadIdx.x; i < U * S; i += kD18Threads) sst[i] = part_ml[slot(i / S, i % S)];
  __syncthreads();
  for (int u = threadIdx.x; u < U; u += kD18Threads) {
    float M = -INFINITY, Mc = -INFINITY;
    for (int sp = 0; sp < S; ++sp) {
      M = fmaxf(M, sst[u * S + sp].x);
      Mc = fmaxf(Mc, sst[u * S + sp].z);
    }
    float L = 0.f, Lc = 0.f;
    for (int sp = 0; sp < S; ++sp) {
      const float4 st = sst[u * S + sp];
      const float f = rescale(st.x, M);
      fac[u * S + sp] = f;
      L += st.y * f;
      Lc += st.w * rescale(st.z, Mc);
    }
    ust[u] = make_float4(M, L, Mc, Lc);
  }
  __syncthreads();
  if (wv == 0) {
    const int d = lane;
    const bool has = d < n_docs;
    const float4 st = has ? ust[d] : make_float4(-INFINITY, 0.f, -INFINITY, 0.f);
    const float r = st.w > 0.f ? st.z * kLn2 + logf(st.w) : -INFINITY;
    float w;
    if (force >= 0) {
      w = d == force ? 1.f : 0.f;
    } else if (wfix) {
      w = has ? wfix[d] : 0.f;
    } else {
      const float logit = beta * r;
      bool keep = has;
      if (top_k > 0 && top_k < n_docs) {
        // Rank by (logit, lower index first) over 64-bit order keys, as the routing top-k does.
        const unsigned long long key =
            has ? ((unsigned long long)order_key(logit) << 32) | (unsigned)~d : 0ull;
        const unsigned hi = (unsigned)(key >> 32), lo = (unsigned)key;
        int rank = 0;
        for (int j = 0; j < n_docs; ++j) {
          const unsigned long long kj = ((unsigned long long)(unsigned)__shfl((int)hi, j) << 32) |
                                        (unsigned)__shfl((int)lo, j);
          rank += kj > key ? 1 : 0;
        }
        keep = has && rank < top_k;
      }
      const float mx = wave_max(keep ? logit : -INFINITY);
      const float e = keep ? expf(logit - mx) : 0.f;
      w = e / wave_sum(e);
    }
    if (has) {
      if (blockIdx.y == 0) {
        const long long o = (((long long)h * G + g) * T + t) * n_docs + d;
        w_out[o] = w;
        r_out[o] = r;
        rmax_out[o] = st.w > 0.f ? st.z * kLn2 : -INFINITY;
      }
      wl[d] = w;
    }
  }
  // Wave wv: the split sums of units wv, wv + 4, ... for dim e (in split order), all S loads of
  // two units in flight.
  const int e = blockIdx.y * kD18MergeDims + lane;
  const int ec = min(e, hd - 1);   // lanes past hd load a valid dim and store nothing
  for (int u0 = wv; u0 < U; u0 += 2 * kD18Waves) {
    const int u1 = u0 + kD18Waves;
    const bool two = u1 < U;   // wave-uniform
    float v0[kD18MaxSplits], v1[kD18MaxSplits];
#pragma unroll
    for (int sp = 0; sp < kD18MaxSplits; ++sp) {
      v0[sp] = sp < S ? part_acc[slot(u0, sp) * hd + ec] : 0.f;
      v1[sp] = two && sp < S ? part_acc[slot(u1, sp) * hd + ec] : 0.f;
    }
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int sp = 0; sp < kD18MaxSplits; ++sp)
      if (sp < S) a0 = fmaf(v0[sp], fac[u0 * S + sp], a0);
    ua[u0][lane] = a0;
    if (two) {
#pragma unroll
      for (int sp = 0; sp < kD18MaxSplits; ++sp)
        if (sp < S) a1 = fmaf(v1[sp], fac[u1 * S + sp], a1);
      ua[u1][lane] = a1;
    }
  }
  __syncthreads();   // ua and wl complete
  if (wv == 0 && e < hd) {
    const float4 so = ust[n_docs];
    const float ao = ua[n_docs][lane];
    float o = 0.f;
    for (int d = 0; d < n_docs; ++d) {
      const float4 sd = ust[d];
      const float M = fmaxf(sd.x, so.x);
      const float a = rescale(sd.x, M), b = rescale(so.x, M);
      o = fmaf(wl[d], (ua[d][lane] * a + ao * b) / (sd.y * a + so.y * b), o);
    }
    out[((long long)t * hq + (long long)h * G + g) * hd + e] = o;
  }
}

size_t d18_align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace
}  // namespace xenc

using namespace xenc;

extern "C" size_t xenc_d18_workspace_bytes(int T, int hq, int n_docs, int hd, int nsplit) {
  if (T < 0 || hq <= 0 || n_docs <= 0 || hd <= 0 || nsplit <= 0) return 0;
  const size_t units = (size_t)T * hq * (n_docs + 1) * nsplit;
  return d18_align256(units * sizeof(float4)) + d18_align256(units * hd * sizeof(float));
}

extern "C" int xenc_d18_read(int dtype, int T, int hq, int hkv, int hd, int n_docs, const float* qd,
                             const float* qo, const void* k_docs, const void* v_docs, long long s_dh,
                             long long s_dn, const int* doc_ptr, const float* k_own, const float* v_own,
                             long long s_oh, long long s_on, int P, float scale, int skip, float beta,
                             int top_k, int force, const float* wfix, int nsplit, float* out, float* w,
                             float* r, float* rmax, void* workspace, size_t workspace_bytes, void* stream) {
  if (dtype < 0 || dtype > 2) return XENC_EINVAL;
  if (T < 0 || P < 0 || skip < 0 || top_k < 0 || hkv <= 0 || hq <= 0 || hq % hkv != 0) return XENC_EINVAL;
  if (hq / hkv > kD18MaxG || n_docs < 1 || n_docs > kD18MaxDocs || force >= n_docs || force < -1)
    return XENC_EINVAL;
  if (nsplit < 1 || nsplit > kD18MaxSplits) return XENC_EINVAL;
  // hd in {32, 64, 128, 256}: a key row is hd / EPL lanes, a power of two <= 64, for the 16-bit
  // document keys (EPL 8) and the fp32 own rows (EPL 4) alike.
  if (hd != 32 && hd != 64 && hd != 128 && hd != 256) return XENC_EINVAL;
  const int epl = dtype == 2 ? 4 : 8;
  if (s_dh % epl || s_dn % epl || s_oh % 4 || s_on % 4) return XENC_EALIGN;
  if (T == 0) return XENC_OK;
  if (!qd || !qo || !k_docs || !v_docs || !doc_ptr || !k_own || !v_own || !out || !w || !r || !rmax)
    return XENC_ENULL;
  if (!aligned16(qd) || !aligned16(qo) || !aligned16(k_docs) || !aligned16(v_docs) || !aligned16(k_own) ||
      !aligned16(v_own))
    return XENC_EALIGN;
  if (!workspace) return XENC_ENULL;
  if (workspace_bytes < xenc_d18_workspace_bytes(T, hq, n_docs, hd, nsplit)) return XENC_EWORKSPACE;
  if ((long long)T * hq > 0x7fffffffLL) return XENC_EINVAL;
  const size_t units = (size_t)T * hq * (n_docs + 1) * nsplit;
  float4* part_ml = static_cast<float4*>(workspace);
  float* part_acc = reinterpret_cast<float*>(static_cast<char*>(workspace) + d18_align256(units * sizeof(float4)));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(T * hkv), (unsigned)((n_docs + 1) * nsplit));
  const float sl2 = scale * kLog2e;
  // Query heads per kv head padded to 1, 2, 4 or 8 (padded heads have q = 0 and are not written).
  const int G = hq / hkv, GP = G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : 8;
#define XENC_D18_LAUNCH(TD, HDV, GPV)                                                              \
  hipLaunchKernelGGL((d18_partials_kernel<TD, HDV, GPV>), grid, dim3(kD18PartThreads), 0, st, hq, hkv, \
                     n_docs, nsplit, qd, qo, static_cast<const TD*>(k_docs),                         \
                     static_cast<const TD*>(v_docs), s_dh, s_dn, doc_ptr, k_own, v_own, s_oh, s_on, P, \
                     T, sl2, skip, part_ml, part_acc)
#define XENC_D18_GP(TD, HDV)                            \
  switch (GP) {                                         \
    case 1: XENC_D18_LAUNCH(TD, HDV, 1); break;         \
    case 2: XENC_D18_LAUNCH(TD, HDV, 2); break;         \
    case 4: XENC_D18_LAUNCH(TD, HDV, 4); break;         \
    default: XENC_D18_LAUNCH(TD, HDV, 8); break;        \
  }
#define XENC_D18_HD(TD)                                  \
  switch (hd) {                                          \
    case 32: XENC_D18_GP(TD, 32) break;                  \
    case 64: XENC_D18_GP(TD, 64) break;                  \
    case 128: XENC_D18_GP(TD, 128) break;                \
    default: XENC_D18_GP(TD, 256) break;                 \
  }
  switch (dtype) {
    case 0: XENC_D18_HD(_Float16) break;
    case 1: XENC_D18_HD(__bf16) break;
    default: XENC_D18_HD(float) break;
  }
#undef XENC_D18_HD
#undef XENC_D18_GP
#undef XENC_D18_LAUNCH
  hipLaunchKernelGGL(d18_merge_kernel, dim3((unsigned)(T * hq), (unsigned)((hd + kD18MergeDims - 1) / kD18MergeDims)),
                     dim3(kD18Threads), 0, st, T, hq, hkv, hd,
                     n_docs, nsplit, part_ml, part_acc, beta, top_k, force, wfix, out, w, r, rmax);
  return check_launch();
}
