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
// `skip`.  Scores of 16 keys x the G heads are MFMA tiles (the query split into parts so that
// the products keep fp32 accuracy: bf16 keys as stored against three bf16 parts of the query,
// fp16 / fp32 keys against fp16 hi + lo); for 16-bit values P.V runs on the matrix cores too (the
// weights split into parts the same way), for the fp32 own rows on the VALU; the running max
// moves only by steps of more than 2^8, so most tiles skip the accumulator rescale; the 4 waves
// merge through LDS in a fixed order.  d18_merge_kernel: one workgroup per (row, query head, 16
// output dims), one unit per 16-lane row, merges the splits (each split's state and accumulator
// requested in one round of loads), joins each document with the own rows (o_d), forms r, rmax
// and the routing weights, and sums w_d o_d.  (Merging where the splits are produced, by the last workgroup of a unit and of a
// row to arrive on a counter, measured slower: each level adds an L2 write-back, an atomic and
// two rounds of loads to the critical path.)  Deterministic: every sum runs in a fixed order.
#include <algorithm>

#include "xenc_common.h"

namespace xenc {
namespace {

constexpr int kD18Threads = 256;   // one wave per SIMD (512 threads cap a wave at 256 registers
                                   // and spill)
constexpr int kD18Waves = kD18Threads / kWave;
constexpr int kD18MaxG = 8;
constexpr int kD18MaxHd = 256;
constexpr int kD18MaxDocs = 64;
constexpr int kD18MaxSplits = 32;
constexpr int kD18BufWord3 = 0x00020000;   // raw buffer descriptor word 3 (b128 loads ignore format)

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

// 2^(m - M) with m = -inf (an empty state) -> 0, also when M = -inf.
__device__ __forceinline__ float rescale(float m, float M) {
  return m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
}

typedef _Float16 d18_half8 __attribute__((ext_vector_type(8)));
typedef __bf16 d18_bf8 __attribute__((ext_vector_type(8)));
constexpr int kD18Tile = 16;   // keys per score tile (the MFMA's 16 rows)

constexpr float kD18Lazy = 8.f;   // log2 headroom of the running max (weights <= 2^8)

// Staged rows in LDS, in 4-byte words.  Every row starts 16-byte aligned, so the MFMA operand
// reads and the row stores are single 16-byte LDS accesses.  The paddings make them free of bank
// conflicts on gfx950 (measured: a row stride of 8 or 24 words mod 64 for the 16-byte reads
// of row lane % 16 at word 4 (lane / 16); 4 or 12 mod 16 for the 4-byte V reads of row
// 4 (lane / 16) + r at word lane % 16):
//   16-bit keys: K rows of HD / 2 + 8 words, then the V rows of HD / 2 + 4 words;
//   fp32 keys:   K rows of HD + 4 words (the V rows stay in registers);
//   the query parts: rows of kD18MaxHd + 16 halves.
template <typename TK, int HD> constexpr int kD18KStride = sizeof(TK) == 4 ? HD + 4 : HD / 2 + 8;
template <int HD> constexpr int kD18VStride = HD / 2 + 4;
template <int HD> constexpr int kD18VBase = kD18Tile * kD18KStride<__bf16, HD>;
constexpr int kD18WaveWords = kD18Tile * (kD18MaxHd + 12);   // covers both layouts at HD 256
constexpr int kD18QRow = kD18MaxHd + 16;
static_assert(kD18VBase<kD18MaxHd> + kD18Tile * kD18VStride<kD18MaxHd> <= kD18WaveWords, "16-bit K and V rows");
static_assert(kD18Tile * kD18KStride<float, kD18MaxHd> <= kD18WaveWords, "fp32 K rows");

// LDS of a partials workgroup: the query fragments (the parts of the 16 padded heads' rows: bf16
// keys three bf16 parts, other keys fp16 hi / lo), per wave the raw key (and 16-bit value) rows of
// its current tile and the tile's probabilities [key][head] with the heads' rescale factors, then
// per wave and query head the state (m, l, mc, lc) and the accumulator.
struct alignas(16) D18Lds {
  unsigned short q[3][16][kD18QRow];
  unsigned kv[kD18Waves][kD18WaveWords];
  float p[kD18Waves][kD18Tile][16];
  float alpha[kD18Waves][16];
  float st[kD18Waves][kD18MaxG][4];
  float acc[kD18Waves][kD18MaxG][kD18MaxHd];
};

// x = hi + lo in fp16 with |x - hi - lo| <= 2^-22 |x| (for |x| in fp16's normal range).
__device__ __forceinline__ _Float16 f16_hi(float x) { return (_Float16)x; }
__device__ __forceinline__ _Float16 f16_lo(float x) { return (_Float16)(x - (float)(_Float16)x); }

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct D18Args {
  int T, hq, hkv, n_docs, S, P, skip, top_k, force;
  float scale_log2, beta;
  const float* qd;
  const float* qo;
  const void* kd;
  const void* vd;
  long long s_dh, s_dn;
  const float* ko;
  const float* vo;
  long long s_oh, s_on;
  const float* wfix;
  f32x4_t* part_ml;      // [T][hkv][D + 1][S][G] (m, l, mc, lc)
  float* part_acc;       // [T][hkv][D + 1][S][G][hd]
  float* out;            // [T][hq][hd]
  float* w;              // w, r, rmax: [hkv][G][T][D]
  float* r;
  float* rmax;
};

// The query rows of the 16 padded heads in chunks of 8 dims: chunk c = thread + 256 j is head
// c / (HD / 8), dims 8 (c % (HD / 8)) .. + 7.  Heads 8 .. 15 are padding (G <= 8), so only the
// chunks c < HD carry values: a thread loads at most one chunk (HD <= 256), from head
// min(g, G - 1) so the loads are unconditional; store_q writes heads past G as 0.
template <int HD>
__device__ __forceinline__ void load_q(const float* __restrict__ q, int G, f32x4_t (&qv)[2]) {
  constexpr int CPR = HD / 8;
  const int c = min((int)threadIdx.x, HD - 1);
  const int g = c / CPR, e0 = (c % CPR) * 8;
  const f32x4_t* src = reinterpret_cast<const f32x4_t*>(q + min(g, G - 1) * HD + e0);
  qv[0] = src[0];
  qv[1] = src[1];
}

// The query rows, scaled to the log2 domain, into LDS (heads past G: 0): the B operand of the
// scores, read by every wave.  For bf16 keys three bf16 parts (q = p0 + p1 + p2 to 2^-24 |q|), so
// the bf16 keys enter the matrix cores as stored; for fp16 / fp32 keys fp16 hi + lo.  One 16-byte
// store per part and chunk.
template <typename TK, int HD>
__device__ __forceinline__ void store_q(const f32x4_t (&qv)[2], int G, float scale_log2, D18Lds& lds) {
  constexpr int CPR = HD / 8, NCH = 16 * CPR;
#pragma unroll
  for (int j = 0; j * kD18Threads < NCH; ++j) {
    const int c = j * kD18Threads + (int)threadIdx.x;
    if (c >= NCH) break;
    const int g = c / CPR, e0 = (c % CPR) * 8;
    const bool live = c < HD && g < G;   // c < HD: this thread's loaded chunk (j = 0)
    unsigned w[3][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      unsigned short h[3][2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const float x = live ? qv[(2 * i + s) / 4][(2 * i + s) % 4] * scale_log2 : 0.f;
        if constexpr (__is_same(TK, __bf16)) {
          const __bf16 p0 = (__bf16)x;
          const float r1 = x - (float)p0;
          const __bf16 p1 = (__bf16)r1;
          h[0][s] = __builtin_bit_cast(unsigned short, p0);
          h[1][s] = __builtin_bit_cast(unsigned short, p1);
          h[2][s] = __builtin_bit_cast(unsigned short, (__bf16)(r1 - (float)p1));
        } else {
          h[0][s] = __builtin_bit_cast(unsigned short, f16_hi(x));
          h[1][s] = __builtin_bit_cast(unsigned short, f16_lo(x));
          h[2][s] = 0;
        }
      }
#pragma unroll
      for (int p = 0; p < 3; ++p) w[p][i] = (unsigned)h[p][0] | ((unsigned)h[p][1] << 16);
    }
    constexpr int NP = __is_same(TK, __bf16) ? 3 : 2;
#pragma unroll
    for (int p = 0; p < NP; ++p)
      *reinterpret_cast<u32x4_t*>(&lds.q[p][g][e0]) = u32x4_t{w[p][0], w[p][1], w[p][2], w[p][3]};
  }
}

// Buffer descriptor over the rows t0 .. t0 + 15 of a split of n rows (row stride s_n elements):
// loads past its last row return 0 without touching memory (none at all when t0 >= n).
template <typename TK, int HD>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const TK* base, long long s_n, int t0, int n) {
  const int nt = min(n - t0, kD18Tile);
  const int bytes = nt > 0 ? (int)(((long long)(nt - 1) * s_n + HD) * (long long)sizeof(TK)) : 0;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<TK*>(base + (long long)max(t0, 0) * s_n), 0, bytes,
                                           kD18BufWord3);
}

// One key split (n keys, the first at index j_base of its unit; n <= 0: empty) for the G query
// heads of a kv head (query rows q [G][HD]), hd = HD.  Wave wv takes the 16-key tiles wv, wv + 4,
// ...  The first tile's K and V rows and the query rows are requested together, so the query's
// latency overlaps the keys'; with 16-bit rows the second tile's rows are requested too.
// Scores on the matrix cores: S^T [16 keys x 16 heads] = K_tile . Q^T with
// v_mfma_f32_16x16x32_f16 (A = keys: lane holds key lane % 16 at dims 32 kb + 8 (lane / 16) + e;
// B = queries: head lane % 16, same dims), q split into fp16 hi + lo (two products; fp32 keys also
// split: three), so the scores keep fp32 accuracy.  Lane (k4 = lane / 16, head = lane % 16) then
// holds the scores of keys 4 k4 .. 4 k4 + 3 for its head: the online softmax per head is an
// in-lane step plus two xor shuffles, and the wave's (m, l) per head is uniform over the wave.
// The probabilities go through LDS to the value lanes: a V row of hd elements is read by
// TPR = HD / EPL lanes (16-byte loads), and acc[g][e] += p[key][g] v[e] in fp32.
// A tile's K and V rows load row-contiguous (16-byte buffer loads, TPR lanes a row): the K rows go
// through LDS into the MFMA layout (loaded in that layout, every 16 lanes would touch 16 rows),
// the V rows stay in registers as loaded.  Rows past n re-read the split's last row (their scores
// are masked).  Keys at unit index >= skip_c (skip_c >= 0) also enter the content max / sum
// (mc, lc).  Writes ml_out[g] = (m, l, mc, lc) (log2 domain) and acc_out[g * HD + e]
// (unnormalised).  Ends with the query rows staged and every wave past the tiles.
template <typename TK, int HD, int GP>
__device__ __forceinline__ void d18_unit(int G, const TK* __restrict__ K, const TK* __restrict__ V, long long s_n,
                                         int n, int j_base, int skip_c, const float* __restrict__ q,
                                         float scale_log2, f32x4_t* __restrict__ ml_out,
                                         float* __restrict__ acc_out, D18Lds& lds) {
  constexpr int EPL = D18Elem<TK>::EPL;
  constexpr int TPR = HD / EPL;              // lanes per row: a power of two <= 64
  constexpr int KPI = kWave / TPR;           // rows per wave load
  constexpr int NI = kD18Tile / KPI > 0 ? kD18Tile / KPI : 1;   // loads per tile (K or V)
  constexpr int KB = HD / 32;                // MFMA k steps
  constexpr bool kF32 = sizeof(TK) == 4;
  constexpr bool kPvMfma = !kF32;            // 16-bit values: P.V on the matrix cores
  static_assert(KPI <= kD18Tile, "a tile holds at least one wave load of rows");
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int hs = lane % 16, k4 = lane / 16;              // score layout
  const bool hi16 = (lane & 16) != 0, hi32 = (lane & 32) != 0;   // halves of the permlane swaps
  const int grp = lane / TPR, e0 = (lane % TPR) * EPL;   // load / value layout
  const int w0 = e0 * (int)sizeof(TK) / 4;               // this lane's first word of a row
  constexpr int KS = kD18KStride<TK, HD>;               // staged K row stride (words)
  unsigned* const kvw = lds.kv[wv];                      // this wave's staged rows
  float acc[GP][EPL];       // VALU P.V: heads x this lane's EPL dims
  f32x4_t accm[HD / 16];    // MFMA P.V: block b, heads 4 k4 .. + 3 at dim 32 (b / 2) + 2 hs + b % 2
#pragma unroll
  for (int g = 0; g < GP; ++g)
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
#pragma unroll
  for (int b = 0; b < HD / 16; ++b) accm[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f, mc = -INFINITY, lc = 0.f;   // head hs
  float mt = -INFINITY;   // the exact max of head hs's scores (m trails it by < 2^8)
  // Content statistics of the split: none (own rows, or every key before skip_c), all (every key
  // at or past skip_c: then they equal (m, l) and are copied at the end), or per key (the split
  // that holds key skip_c).  Workgroup-uniform.
  const int cmode = skip_c < 0 || j_base + n <= skip_c ? 0 : j_base >= skip_c ? 1 : 2;
  // Rows t0 .. t0 + 15 (clamped to the tile's last row); unconditional, in bounds by the descriptor.
  auto load_rows = [&](const TK* base, int t0, u32x4_t (&r)[NI]) {
    const __amdgpu_buffer_rsrc_t rs = tile_rsrc<TK, HD>(base, s_n, t0, n);
    const int last = max(min(n - t0, kD18Tile) - 1, 0);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const unsigned off = (unsigned)(((long long)min(i * KPI + grp, last) * s_n + e0) * (long long)sizeof(TK));
      r[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
    }
  };
  // One 16-key tile (its K and V rows in kr, vr; keys t0 .. t0 + 15 of the split).
  auto tile = [&](const u32x4_t (&kr)[NI], const u32x4_t (&vr)[NI], int t0) {
    // The tile's K rows to LDS (16-bit keys: then the V rows).
#pragma unroll
    for (int i = 0; i < NI; ++i) *reinterpret_cast<u32x4_t*>(&kvw[(i * KPI + grp) * KS + w0]) = kr[i];
    if constexpr (kPvMfma) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
        *reinterpret_cast<u32x4_t*>(&kvw[kD18VBase<HD> + (i * KPI + grp) * kD18VStride<HD> + w0]) = vr[i];
    }
    wave_sync_lds();
    // One accumulator per product, so the MFMA chains are independent; summed at the end.
    f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0, s2 = s0;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int qo = 32 * kb + 8 * k4;
      if constexpr (__is_same(TK, __bf16)) {
        const d18_bf8 kv = *reinterpret_cast<const d18_bf8*>(&kvw[hs * KS + qo / 2]);
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, *reinterpret_cast<const d18_bf8*>(&lds.q[0][hs][qo]), s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, *reinterpret_cast<const d18_bf8*>(&lds.q[1][hs][qo]), s1, 0, 0, 0);
        s2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, *reinterpret_cast<const d18_bf8*>(&lds.q[2][hs][qo]), s2, 0, 0, 0);
      } else {
        const d18_half8 qh = *reinterpret_cast<const d18_half8*>(&lds.q[0][hs][qo]);
        const d18_half8 ql = *reinterpret_cast<const d18_half8*>(&lds.q[1][hs][qo]);
        if constexpr (kF32) {
          const f32x4_t a = *reinterpret_cast<const f32x4_t*>(&kvw[hs * KS + qo]);
          const f32x4_t b = *reinterpret_cast<const f32x4_t*>(&kvw[hs * KS + qo + 4]);
          d18_half8 ka, kl;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            ka[e] = f16_hi(a[e]);
            kl[e] = f16_lo(a[e]);
            ka[4 + e] = f16_hi(b[e]);
            kl[4 + e] = f16_lo(b[e]);
          }
          s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh, s0, 0, 0, 0);
          s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql, s1, 0, 0, 0);
          s2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh, s2, 0, 0, 0);
        } else {
          const d18_half8 ka = *reinterpret_cast<const d18_half8*>(&kvw[hs * KS + qo / 2]);
          s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh, s0, 0, 0, 0);
          s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql, s1, 0, 0, 0);
        }
      }
    }
    const f32x4_t sc = (s0 + s1) + s2;
    // Online softmax of head hs over the tile's keys t0 + 4 k4 + r.
    bool ok[4];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      ok[r] = t0 + 4 * k4 + r < n;
      if (ok[r]) mx = fmaxf(mx, sc[r]);
    }
    mx = fmaxf(mx, swap_partner<16>(mx, hi16));
    mx = fmaxf(mx, swap_partner<32>(mx, hi32));
    // The running max moves only when the tile's max passes it by more than 2^8: the weights stay
    // <= 256 and most tiles need no rescale of the accumulators (the state (m, l, acc) stays exact:
    // a rescale is a power of two).
    const float mn = mx > m + kD18Lazy ? mx : m;
    mt = fmaxf(mt, mx);
    const float a = rescale(m, mn);
    const bool any_rescale = __ballot(m != -INFINITY && mn != m) != 0;   // wave-uniform
    float pr[4], ps = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pr[r] = ok[r] ? __builtin_amdgcn_exp2f(sc[r] - mn) : 0.f;
      ps += pr[r];
    }
    ps += swap_partner<16>(ps, hi16);
    ps += swap_partner<32>(ps, hi32);
    l = l * a + ps;
    m = mn;
    if (cmode == 2) {
      float mcx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (ok[r] && j_base + t0 + 4 * k4 + r >= skip_c) mcx = fmaxf(mcx, sc[r]);
      mcx = fmaxf(mcx, swap_partner<16>(mcx, hi16));
      mcx = fmaxf(mcx, swap_partner<32>(mcx, hi32));
      const float mcn = fmaxf(mc, mcx);
      float cs = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (ok[r] && j_base + t0 + 4 * k4 + r >= skip_c) cs += __builtin_amdgcn_exp2f(sc[r] - mcn);
      cs += swap_partner<16>(cs, hi16);
      cs += swap_partner<32>(cs, hi32);
      lc = lc * rescale(mc, mcn) + cs;
      mc = mcn;
    }
    if constexpr (kPvMfma) {
      // P.V on the matrix cores, v_mfma_f32_16x16x32 (lane l: A row l % 16, B column l % 16, k
      // slots 8 (l / 16) .. + 7): D[head][dim] += sum_k A[head][k] B[k][dim].  This lane's p (head
      // hs, keys 4 k4 + r) fill its A slots as the parts of p: bf16 values [hi, mid] and [lo, 0]
      // (two products, 24 bits of p), fp16 values [hi, lo] (one, 22 bits); the B slots carry the
      // same 4 keys' V at the lane's dim twice.  The 32 dims of pair c are read as 16-bit pairs:
      // lane hs takes dims 32 c + 2 hs (block 2 c) and 32 c + 2 hs + 1 (block 2 c + 1).  D lane l:
      // heads 4 (l / 16) + r.
      if (any_rescale) {
        if (k4 == 0) lds.alpha[wv][hs] = a;
        wave_sync_lds();
        float al[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) al[r] = lds.alpha[wv][4 * k4 + r];
#pragma unroll
        for (int b = 0; b < HD / 16; ++b)
#pragma unroll
          for (int r = 0; r < 4; ++r) accm[b][r] *= al[r];
      }
      u32x4_t a1, a2;   // the A operand parts as packed 16-bit pairs
      if constexpr (__is_same(TK, __bf16)) {
        unsigned hi[4], mid[4], lo[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const __bf16 h = (__bf16)pr[r];
          const float rem = pr[r] - (float)h;
          const __bf16 md = (__bf16)rem;
          hi[r] = __builtin_bit_cast(unsigned short, h);
          mid[r] = __builtin_bit_cast(unsigned short, md);
          lo[r] = __builtin_bit_cast(unsigned short, (__bf16)(rem - (float)md));
        }
        a1 = u32x4_t{hi[0] | hi[1] << 16, hi[2] | hi[3] << 16, mid[0] | mid[1] << 16, mid[2] | mid[3] << 16};
        a2 = u32x4_t{lo[0] | lo[1] << 16, lo[2] | lo[3] << 16, 0u, 0u};
      } else {
        unsigned hi[4], lo[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          hi[r] = __builtin_bit_cast(unsigned short, f16_hi(pr[r]));
          lo[r] = __builtin_bit_cast(unsigned short, f16_lo(pr[r]));
        }
        a1 = u32x4_t{hi[0] | hi[1] << 16, hi[2] | hi[3] << 16, lo[0] | lo[1] << 16, lo[2] | lo[3] << 16};
      }
#pragma unroll
      for (int c = 0; c < HD / 32; ++c) {
        unsigned w[4];   // keys 4 k4 + r, dims 32 c + 2 hs (low half) and + 1 (high half)
#pragma unroll
        for (int r = 0; r < 4; ++r) w[r] = kvw[kD18VBase<HD> + (4 * k4 + r) * kD18VStride<HD> + 16 * c + hs];
        const unsigned ev01 = (w[0] & 0xffffu) | (w[1] << 16), ev23 = (w[2] & 0xffffu) | (w[3] << 16);
        const unsigned od01 = (w[0] >> 16) | (w[1] & 0xffff0000u), od23 = (w[2] >> 16) | (w[3] & 0xffff0000u);
        const u32x4_t be = {ev01, ev23, ev01, ev23}, bo = {od01, od23, od01, od23};
        if constexpr (__is_same(TK, __bf16)) {
          const d18_bf8 x1 = __builtin_bit_cast(d18_bf8, a1), x2 = __builtin_bit_cast(d18_bf8, a2);
          const d18_bf8 ye = __builtin_bit_cast(d18_bf8, be), yo = __builtin_bit_cast(d18_bf8, bo);
          accm[2 * c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1, ye, accm[2 * c], 0, 0, 0);
          accm[2 * c + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1, yo, accm[2 * c + 1], 0, 0, 0);
          accm[2 * c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x2, ye, accm[2 * c], 0, 0, 0);
          accm[2 * c + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x2, yo, accm[2 * c + 1], 0, 0, 0);
        } else {
          const d18_half8 x1 = __builtin_bit_cast(d18_half8, a1);
          accm[2 * c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, __builtin_bit_cast(d18_half8, be), accm[2 * c], 0, 0, 0);
          accm[2 * c + 1] =
              __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, __builtin_bit_cast(d18_half8, bo), accm[2 * c + 1], 0, 0, 0);
        }
      }
    } else {
      // Probabilities and rescale factors to the value lanes.
#pragma unroll
      for (int r = 0; r < 4; ++r) lds.p[wv][4 * k4 + r][hs] = pr[r];
      if (k4 == 0) lds.alpha[wv][hs] = a;
      wave_sync_lds();
      if (any_rescale) {
#pragma unroll
        for (int g = 0; g < GP; ++g) {
          const float ag = lds.alpha[wv][g];
#pragma unroll
          for (int e = 0; e < EPL; ++e) acc[g][e] *= ag;
        }
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
    }
    wave_sync_lds();   // the next tile's keys and probabilities overwrite these
  };
  constexpr int kStep = kD18Waves * kD18Tile;   // a wave's next tile
  const int t_first = wv * kD18Tile;
  f32x4_t qv[2];
  if constexpr (!kF32) {
    // 16-bit rows: two tiles in registers, the next one loading while this one computes (loads
    // past the split return 0 and touch no memory, so every load is unconditional).  The query
    // loads go between the two tiles' loads, so staging the query waits for the first tile only.
    u32x4_t k0[NI], v0[NI], k1[NI], v1[NI];
    load_rows(K, t_first, k0);
    load_rows(V, t_first, v0);
    load_q<HD>(q, G, qv);
    load_rows(K, t_first + kStep, k1);
    load_rows(V, t_first + kStep, v1);
    store_q<TK, HD>(qv, G, scale_log2, lds);
    __syncthreads();
    if (n <= t_first + 2 * kStep) {
      // At most two tiles for this wave (a decode-sized split): straight-line code, so the wait
      // for the second tile's loads comes only before the second tile (in a loop the back edge
      // would make the first tile wait for both).
      if (t_first < n) tile(k0, v0, t_first);
      if (t_first + kStep < n) tile(k1, v1, t_first + kStep);
    } else {
      for (int t0 = t_first; t0 < n; t0 += 2 * kStep) {
        tile(k0, v0, t0);
        load_rows(K, t0 + 2 * kStep, k0);
        load_rows(V, t0 + 2 * kStep, v0);
        if (t0 + kStep >= n) break;
        tile(k1, v1, t0 + kStep);
        load_rows(K, t0 + 3 * kStep, k1);
        load_rows(V, t0 + 3 * kStep, v1);
      }
    }
  } else {
    u32x4_t kr[NI], vr[NI];
    load_rows(K, t_first, kr);
    load_rows(V, t_first, vr);
    load_q<HD>(q, G, qv);
    store_q<TK, HD>(qv, G, scale_log2, lds);
    __syncthreads();
    for (int t0 = t_first; t0 < n; t0 += kStep) {
      if (t0 != t_first) {
        load_rows(K, t0, kr);
        load_rows(V, t0, vr);
      }
      tile(kr, vr, t0);
    }
  }
  if (cmode == 1) {   // every key counts: the content max is the exact max, l rescaled to it
    mc = mt;
    lc = l * rescale(m, mt);
  }
  if constexpr (kPvMfma) {
    // The MFMA sums cover every key of the wave: heads 4 k4 + r (those < G) to LDS.
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (4 * k4 + r < G) {
#pragma unroll
        for (int b = 0; b < HD / 16; ++b) lds.acc[wv][4 * k4 + r][32 * (b / 2) + 2 * hs + (b % 2)] = accm[b][r];
      }
  } else {
    // Lane groups of the wave (same dims, different keys) share the wave's state: their sums add.
#pragma unroll
    for (int o = TPR; o < kWave; o <<= 1)
#pragma unroll
      for (int g = 0; g < GP; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] += shfl_xor(acc[g][e], o);
    if (grp == 0) {
#pragma unroll
      for (int g = 0; g < GP; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) lds.acc[wv][g][e0 + e] = acc[g][e];
    }
  }
  // The 4 waves through LDS, summed in wave order.
  if (lane < G) {
    lds.st[wv][lane][0] = m;
    lds.st[wv][lane][1] = l;
    lds.st[wv][lane][2] = mc;
    lds.st[wv][lane][3] = lc;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < G * HD; i += kD18Threads) {
    const int g = i / HD, e = i % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kD18Waves; ++w) M = fmaxf(M, lds.st[w][g][0]);
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kD18Waves; ++w) s += lds.acc[w][g][e] * rescale(lds.st[w][g][0], M);
    acc_out[i] = s;
  }
  if ((int)threadIdx.x < G) {
    const int g = threadIdx.x;
    float M = -INFINITY, Mc = -INFINITY;
#pragma unroll
    for (int w = 0; w < kD18Waves; ++w) {
      M = fmaxf(M, lds.st[w][g][0]);
      Mc = fmaxf(Mc, lds.st[w][g][2]);
    }
    float L = 0.f, Lc = 0.f;
#pragma unroll
    for (int w = 0; w < kD18Waves; ++w) {
      L += lds.st[w][g][1] * rescale(lds.st[w][g][0], M);
      Lc += lds.st[w][g][3] * rescale(lds.st[w][g][2], Mc);
    }
    ml_out[g] = f32x4_t{M, L, Mc, Lc};
  }
}

// Max over each aligned group of 16 lanes (one row), every lane of the row ending with it (DPP).
__device__ __forceinline__ float row_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));    // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f<0x4E>(v));    // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f<0x141>(v));   // row_half_mirror
  return fmaxf(v, dpp_f<0x140>(v));   // row_mirror
}

// The value of lane N of this lane's 16-lane row (DPP row_newbcast).
template <int N>
__device__ __forceinline__ float row_bcast(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x150 + N, 0xF, 0xF, false));
}

// a += sum over the splits s < S (in split order) of v[s] times the factor of split s, which lane
// s % 16 of the row holds (f0 for s < 16, f1 for s >= 16).
template <int S0>
__device__ __forceinline__ void sum_splits(const float (&v)[kD18MaxSplits], float f0, float f1, int S, float& a) {
  if constexpr (S0 < kD18MaxSplits) {
    if (S0 < S) a = fmaf(v[S0], row_bcast<S0 % 16>(S0 < 16 ? f0 : f1), a);
    sum_splits<S0 + 1>(v, f0, f1, S, a);
  }
}

// Routing weight of document d (lane d; has = d < D) from r: one-hot at force, wfix, or the
// softmax of beta * r over the top_k largest (ties to the lower index, ranked over 64-bit order
// keys as the routing top-k does).  Called by whole waves.
__device__ __forceinline__ float doc_weight(float r, bool has, int d, int D, float beta, int top_k, int force,
                                            const float* __restrict__ wfix) {
  if (force >= 0) return d == force ? 1.f : 0.f;
  if (wfix) return has ? wfix[d] : 0.f;
  const float logit = beta * r;
  bool keep = has;
  if (top_k > 0 && top_k < D) {
    const unsigned long long key = has ? ((unsigned long long)order_key(logit) << 32) | (unsigned)~d : 0ull;
    const unsigned hi = (unsigned)(key >> 32), lo = (unsigned)key;
    int rank = 0;
    for (int j = 0; j < D; ++j) {
      const unsigned long long kj =
          ((unsigned long long)(unsigned)__shfl((int)hi, j) << 32) | (unsigned)__shfl((int)lo, j);
      rank += kj > key ? 1 : 0;
    }
    keep = has && rank < top_k;
  }
  const float mx = wave_max(keep ? logit : -INFINITY);
  const float e = keep ? expf(logit - mx) : 0.f;
  return e / wave_sum(e);
}

// One workgroup of 2 waves per (row t, kv head h, query head g) and block of 16 output dims:
// blockIdx.x = (t * hkv + h) * G + g, blockIdx.y = dim block.  Each 16-lane row of the
// workgroup merges one unit (row k of the 8 takes units k, k + 8, ...): lane j of the row holds
// the states of splits j and j + 16 and the S accumulator values of dim 16 blk + j, all
// requested in one round.  The unit's max M, the factors 2^(m_s - M) and the sums L, Lc come
// from row reductions (a fixed tree); the accumulator sums its splits in split order with the
// factors fetched from the row's lanes.  Wave 0 then forms r, rmax and the routing weights (one
// lane per document; block 0 writes w, r, rmax) and sums o[e] = sum_d w_d o_d[e], o_d the join
// of document d and the own rows: o_d = (a_d acc_d + b_d acc_own) / (a_d L_d + b_d L_own) with
// a_d = 2^(M_d - M), b_d = 2^(M_own - M), M = max(M_d, M_own).
constexpr int kD18MergeDims = 16;
constexpr int kD18MergeThreads = 128;
constexpr int kD18MergeRows = kD18MergeThreads / kD18MergeDims;   // units in flight

__global__ __launch_bounds__(kD18MergeThreads) void d18_merge_kernel(const D18Args A, int hd) {
  __shared__ f32x4_t ust[kD18MaxDocs + 1];                 // per unit: (M, L, Mc, Lc)
  __shared__ float ua[kD18MaxDocs + 1][kD18MergeDims];     // per unit: the merged accumulator
  __shared__ float wl[kD18MaxDocs];
  const int G = A.hq / A.hkv, U = A.n_docs + 1, D = A.n_docs, S = A.S;
  const int g = blockIdx.x % G, th = blockIdx.x / G;
  const int t = th / A.hkv, h = th % A.hkv;
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  const int row = threadIdx.x / kD18MergeDims, j = threadIdx.x % kD18MergeDims;
  const int e = blockIdx.y * kD18MergeDims + j;
  const int ec = min(e, hd - 1);   // lanes past hd load a valid dim and store nothing
  const f32x4_t empty = {-INFINITY, 0.f, -INFINITY, 0.f};
  for (int u0 = 0; u0 < U; u0 += kD18MergeRows) {
    const int u = u0 + row;
    const bool mine = u < U;
    const long long slot0 = ((long long)th * U + min(u, U - 1)) * S * G + g;   // split s at slot0 + s * G
    const f32x4_t s0 = j < S ? A.part_ml[slot0 + (long long)j * G] : empty;
    const f32x4_t s1 = j + 16 < S ? A.part_ml[slot0 + (long long)(j + 16) * G] : empty;
    float v[kD18MaxSplits];
#pragma unroll
    for (int s = 0; s < kD18MaxSplits; ++s) v[s] = s < S ? A.part_acc[(slot0 + (long long)s * G) * hd + ec] : 0.f;
    const float M = row_max(fmaxf(s0[0], s1[0])), Mc = row_max(fmaxf(s0[2], s1[2]));
    const float f0 = rescale(s0[0], M), f1 = rescale(s1[0], M);
    const float L = group_sum<16>(s0[1] * f0 + s1[1] * f1);
    const float Lc = group_sum<16>(s0[3] * rescale(s0[2], Mc) + s1[3] * rescale(s1[2], Mc));
    float a = 0.f;
    sum_splits<0>(v, f0, f1, S, a);
    if (mine) {
      ua[u][j] = a;
      if (j == 0) ust[u] = f32x4_t{M, L, Mc, Lc};
    }
  }
  __syncthreads();
  if (wv != 0) return;
  {
    const int d = lane;
    const bool has = d < D;
    const f32x4_t st = has ? ust[d] : empty;
    const float r = st[3] > 0.f ? st[2] * kLn2 + logf(st[3]) : -INFINITY;
    const float w = doc_weight(r, has, d, D, A.beta, A.top_k, A.force, A.wfix);
    if (has) {
      if (blockIdx.y == 0) {
        const long long o = (((long long)h * G + g) * A.T + t) * D + d;
        A.w[o] = w;
        A.r[o] = r;
        A.rmax[o] = st[3] > 0.f ? st[2] * kLn2 : -INFINITY;
      }
      wl[d] = w;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if (lane < kD18MergeDims && e < hd) {
    const f32x4_t so = ust[D];
    const float ao = ua[D][j];
    float o = 0.f;
    for (int d = 0; d < D; ++d) {
      const f32x4_t sd = ust[d];
      const float M = fmaxf(sd[0], so[0]);
      const float a = rescale(sd[0], M), b = rescale(so[0], M);
      o = fmaf(wl[d], (ua[d][j] * a + ao * b) / (sd[1] * a + so[1] * b), o);
    }
    A.out[((long long)t * A.hq + (long long)h * G + g) * hd + e] = o;
  }
}

// Partials of split s of unit u of (row t, kv head h): blockIdx = (t * hkv + h, u * S + s); u < D
// a document (keys split into S ranges of ceil(N_d / S)), u = D the own rows (S ranges of
// ceil((P + T) / S), cut at row t's causal end P + t + 1).
template <typename TD, int HD, int GP>
__global__ __launch_bounds__(kD18Threads) void d18_partials_kernel(const D18Args A, const int* __restrict__ doc_ptr) {
  __shared__ D18Lds lds;
  const int th = blockIdx.x;
  const int t = th / A.hkv, h = th % A.hkv;
  const int u = blockIdx.y / A.S, sp = blockIdx.y % A.S;
  const int G = A.hq / A.hkv, U = A.n_docs + 1;
  const long long slot = (((long long)th * U + u) * A.S + sp) * G;
  if (u < A.n_docs) {
    const int n0 = doc_ptr[u], N = doc_ptr[u + 1] - n0;
    const int chunk = (N + A.S - 1) / A.S;
    const int lo = sp * chunk, n = min(N - lo, chunk);
    const long long off = (long long)h * A.s_dh + (long long)(n0 + lo) * A.s_dn;
    d18_unit<TD, HD, GP>(G, static_cast<const TD*>(A.kd) + off, static_cast<const TD*>(A.vd) + off, A.s_dn, n, lo,
                         N > A.skip ? A.skip : 0, A.qd + (((long long)u * A.T + t) * A.hq + (long long)h * G) * HD,
                         A.scale_log2, A.part_ml + slot, A.part_acc + slot * HD, lds);
  } else {
    const int chunk = (A.P + A.T + A.S - 1) / A.S;
    const int lo = sp * chunk, n = min(A.P + t + 1 - lo, chunk);
    const long long off = (long long)h * A.s_oh + (long long)lo * A.s_on;
    d18_unit<float, HD, GP>(G, A.ko + off, A.vo + off, A.s_on, n, lo, -1,
                            A.qo + ((long long)t * A.hq + (long long)h * G) * HD, A.scale_log2, A.part_ml + slot,
                            A.part_acc + slot * HD, lds);
  }
}

size_t d18_align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace
}  // namespace xenc

using namespace xenc;

extern "C" size_t xenc_d18_workspace_bytes(int T, int hq, int n_docs, int hd, int nsplit) {
  if (T < 0 || hq <= 0 || n_docs <= 0 || hd <= 0 || nsplit <= 0) return 0;
  const size_t units = (size_t)T * hq * (n_docs + 1) * nsplit;
  return d18_align256(units * sizeof(f32x4_t)) + d18_align256(units * hd * sizeof(float));
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
  if (s_dh % epl || s_dn % epl || s_oh % 4 || s_on % 4 || s_dn < hd || s_on < hd) return XENC_EALIGN;
  if (T == 0) return XENC_OK;
  if (!qd || !qo || !k_docs || !v_docs || !doc_ptr || !k_own || !v_own || !out || !w || !r || !rmax)
    return XENC_ENULL;
  if (!aligned16(qd) || !aligned16(qo) || !aligned16(k_docs) || !aligned16(v_docs) || !aligned16(k_own) ||
      !aligned16(v_own) || !aligned16(out))
    return XENC_EALIGN;
  if (!workspace) return XENC_ENULL;
  if (!aligned16(workspace)) return XENC_EALIGN;
  if (workspace_bytes < xenc_d18_workspace_bytes(T, hq, n_docs, hd, nsplit)) return XENC_EWORKSPACE;
  if ((long long)T * hkv > 0x7fffffffLL) return XENC_EINVAL;
  // A 16-row tile's bytes fit the 32-bit buffer descriptor.
  const long long esz = dtype == 2 ? 4 : 2;
  if ((15 * s_dn + hd) * esz > 0x7fffffffLL || (15 * s_on + hd) * 4 > 0x7fffffffLL) return XENC_EINVAL;
  const size_t units = (size_t)T * hq * (n_docs + 1) * nsplit;
  char* ws = static_cast<char*>(workspace);
  D18Args A;
  A.T = T;
  A.hq = hq;
  A.hkv = hkv;
  A.n_docs = n_docs;
  A.S = nsplit;
  A.P = P;
  A.skip = skip;
  A.top_k = top_k;
  A.force = force;
  A.scale_log2 = scale * kLog2e;
  A.beta = beta;
  A.qd = qd;
  A.qo = qo;
  A.kd = k_docs;
  A.vd = v_docs;
  A.s_dh = s_dh;
  A.s_dn = s_dn;
  A.ko = k_own;
  A.vo = v_own;
  A.s_oh = s_oh;
  A.s_on = s_on;
  A.wfix = wfix;
  A.part_ml = reinterpret_cast<f32x4_t*>(ws);
  A.part_acc = reinterpret_cast<float*>(ws + d18_align256(units * sizeof(f32x4_t)));
  A.out = out;
  A.w = w;
  A.r = r;
  A.rmax = rmax;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(T * hkv), (unsigned)((n_docs + 1) * nsplit));
  // Query heads per kv head padded to 1, 2, 4 or 8 (padded heads have q = 0 and are not written).
  const int G = hq / hkv, GP = G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : 8;
#define XENC_D18_LAUNCH(TD, HDV, GPV) \
  hipLaunchKernelGGL((d18_partials_kernel<TD, HDV, GPV>), grid, dim3(kD18Threads), 0, st, A, doc_ptr)
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
                     dim3(kD18MergeThreads), 0, st, A, hd);
  return check_launch();
}
