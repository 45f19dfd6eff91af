// Prefill / registration read of the Library on MFMA (fp16 operands, fp32 accumulation), and its
// dQ backward.  Many query rows read the same library (a training step or a long prompt), so the
// read is a dense contraction:
//
//   forward   S^T[n, t] = K_c[n] . q_t                 (scores kernel, MFMA, one chunk per tile)
//             p[t, c, n] = softmax_n(read_temp * S)     (epilogue: masked per-chunk softmax)
//             r[t]       = sum_c w[t,c] sum_n p K_c[n]  (readout kernel, MFMA)
//   backward  U^T[n, t] = K_c[n] . g_t                 (scores kernel, MFMA)
//             gamma[t,c] = sum_n p U ;  dS = read_temp * w p (U - gamma)   (epilogue)
//             dq_read[t] = sum_{c,n} dS K_c[n]         (readout kernel)
//             dq_route   = route_temp * sum_c w (dw - sum w dw) S_c, dw = gamma + dL/dw (route bwd)
// This is the math of LibraryInjector._branch (xenc/injector.py:236-265) and of its autograd
// (scripts/register_doc.py:699), with K = V tied.
//
// Layouts.  The library is resident across many calls, so each page is also kept in two
// fragment-ordered copies built once (xenc_fragment_pages): in these, the 64 lanes' MFMA
// fragments of one (32-row, 16-column) block are one contiguous 1 KiB, so every fragment load of
// the operand that a wave owns alone is a single coalesced read.
//   layout A [P][N/32][d/16][64][8]: lane l of block (sg, kb) = K[32sg + l%32][16kb + 8(l/32) + e]
//   layout B [P][d/32][N/16][64][8]: lane l of block (db, nb) = K[16nb + 8(l/32) + e][32db + l%32]
// The probabilities p and the backward dS are stored octet-major, [C*N/8][M][8] (8 slots of a
// row in 16 bytes, rows fastest), so the scores epilogue writes 512 contiguous bytes per
// instruction and the readout stages them with contiguous row loads.  The scores epilogues store
// them (and the backward's reads p) nontemporally: each element passes there once, and the L2
// keeps the page fragments and query rows the XCD's other tiles reuse.
//
// The scores tile covers a whole chunk (512 slots) x 128 query rows, so the chunk softmax is
// local to the workgroup; S^T is formed (slots as the MFMA M dimension) so that each lane holds 32
// slot scores of 4 query rows: the softmax over slots is an in-lane reduction plus one xor-32
// shuffle plus an 8-wave LDS exchange.
#include <algorithm>
#include <climits>

#include "xenc_common.h"

namespace xenc {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int BK = 64;              // k (d or slot) columns per main-loop step: four MFMA k16 steps
constexpr int kRowsPerTile = 128;   // query rows per scores tile
constexpr int kSlotsPerTile = 512;  // slots per scores tile (a whole page)
constexpr int kReadoutRows = 128;   // query rows per readout tile

// LDS tiles hold rows of BK = 64 halves (128 B = 8 chunks of 16 B).  Chunk c of row r sits at
// position c ^ ((r ^ (r >> 3)) & 7): the 8 (or 16) rows that one ds_read_b128 fragment load
// serves per cycle then fall on disjoint banks, for 32 and for 64 banks alike.
__device__ __forceinline__ int swz(int r, int c) { return r * BK + ((c ^ ((r ^ (r >> 3)) & 7)) << 3); }

__device__ __forceinline__ f32x16 mfma32(const half8_t& a, const half8_t& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Instruction classes of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008, kSchedVmemRead = 0x020, kSchedDsRead = 0x100;

// One 16-byte chunk per lane from global memory straight into LDS (gfx950
// global_load_lds_dwordx4): lane i of the wave writes lds_wave_base + 16 i.  lds_wave_base must
// be wave-uniform.  Issued as inline assembly so that the compiler does not treat the LDS
// write as pending at every barrier and LDS read (it would wait for every outstanding global
// load there); the caller waits for these loads itself (wait_vmem) before publishing the LDS.
__device__ __forceinline__ void stage_to_lds(_Float16* lds_wave_base, const _Float16* src) {
  const unsigned lds = __builtin_amdgcn_readfirstlane(
      (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void*)lds_wave_base);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(src) : "memory", "m0");
}

// Wait until at most N vector-memory operations of this wave are outstanding (they complete in
// issue order for the counter).
template <int N>
__device__ __forceinline__ void wait_vmem() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

constexpr int kChunkGroup = 4;  // scores tiles: chunks per group, all row tiles of a group adjacent

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
// fp32 -> fp16 rows: y [M, d] (contiguous) from x [M, ldx].  A workgroup converts whole rows
// (rows blockIdx.x, + gridDim.x, ...); each thread issues the loads of up to kCastPer groups of 4
// elements of a row before it converts and stores them.
constexpr int kCastThreads = 256, kCastPer = 4;
__global__ __launch_bounds__(kCastThreads) void cast_rows_f16_kernel(const float* __restrict__ x,
                                                                     long long ldx, int M, int d,
                                                                     _Float16* __restrict__ y) {
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  const int n4 = d / 4;
  for (int row = blockIdx.x; row < M; row += gridDim.x) {
    const float* xr = x + (long long)row * ldx;
    _Float16* yr = y + (long long)row * d;
    for (int c0 = threadIdx.x; c0 < n4; c0 += kCastThreads * kCastPer) {
      f32x4v v[kCastPer];
#pragma unroll
      for (int u = 0; u < kCastPer; ++u) {
        const int cc = c0 + u * kCastThreads;
        if (cc < n4) v[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4v*>(xr + 4 * cc));
      }
#pragma unroll
      for (int u = 0; u < kCastPer; ++u) {
        const int cc = c0 + u * kCastThreads;
        if (cc < n4) {
          const half4_t h = {(_Float16)v[u][0], (_Float16)v[u][1], (_Float16)v[u][2], (_Float16)v[u][3]};
          __builtin_nontemporal_store(h, reinterpret_cast<half4_t*>(yr + 4 * cc));
        }
      }
    }
  }
}

// pages [P, N, d] -> a fragment-ordered copy (layout A or B above); one thread per lane-chunk.
template <int LAYOUT>
__global__ __launch_bounds__(256) void fragment_pages_kernel(const _Float16* __restrict__ pages,
                                                             long long P, int N, int d,
                                                             _Float16* __restrict__ out) {
  const long long total = P * (long long)N * d / 8;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const int lane = (int)(i & 63);
    const long long blk = i >> 6;
    half8_t v;
    if (LAYOUT == 0) {  // [P][N/32][d/16][64][8]
      const int nkb = d / 16, nsg = N / 32;
      const int kb = (int)(blk % nkb), sg = (int)((blk / nkb) % nsg);
      const long long p = blk / ((long long)nkb * nsg);
      const _Float16* src = pages + (p * N + 32 * sg + (lane & 31)) * d + 16 * kb + 8 * (lane >> 5);
      v = *reinterpret_cast<const half8_t*>(src);
    } else {            // [P][d/32][N/16][64][8]
      const int nnb = N / 16, ndb = d / 32;
      const int nb = (int)(blk % nnb), db = (int)((blk / nnb) % ndb);
      const long long p = blk / ((long long)nnb * ndb);
      const _Float16* src = pages + (p * N + 16 * nb + 8 * (lane >> 5)) * d + 32 * db + (lane & 31);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = src[(long long)e * d];
    }
    *reinterpret_cast<half8_t*>(out + i * 8) = v;
  }
}

// ------------------------------------------------------------------------------------------
// Scores kernel: one workgroup = (library g, 128-row tile, chunk c), 8 waves; wave w owns slots
// [64w, 64w+64) (two 32-row MFMA tiles) x all 128 rows (four 32-column tiles).  The slot rows of
// a wave are private to it: their fragments come straight from the layout-A page copy (one
// coalesced 1 KiB load each), refilled for the next k-step as soon as they are consumed; the 128
// query rows are shared by all waves and staged through LDS (three swizzled stages, one barrier
// per k-step).
// MODE 0 (forward): writes p = masked softmax over the chunk's slots (fp16, octet-major), and
//                    when gamma is given gamma[t, c] = log-sum-exp of the row's scaled scores.
// MODE 1 (backward): reads p, writes dS = read_temp * w[t,c] * p * (U - gamma) (octet-major)
//                    and gamma[t, c] = sum_n p U.
// MODE 2 (forward, linear read): writes p = S / sqrt(n_valid) on valid slots, 0 on the others.
// MODE 3 (backward, linear read): reads p, writes dS = w[t,c] * U / sqrt(n_valid) (0 on masked
//                    slots) and gamma[t, c] = sum_n p U.
template <int MODE>
__global__ __launch_bounds__(512) void scores_kernel(
    const _Float16* __restrict__ X, int d, const int* __restrict__ row_ptr,
    const int* __restrict__ tile_ptr, int G, const _Float16* __restrict__ pages_a, int N,
    long long page_stride, const int* __restrict__ chunk_ptr, const int* __restrict__ chunk_page,
    const int* __restrict__ chunk_nvalid, float temp, const float* __restrict__ w, long long ldw,
    _Float16* __restrict__ P, long long p_rows, _Float16* __restrict__ dS,
    float* __restrict__ gamma, long long ldg) {
  __shared__ _Float16 lB[3][kRowsPerTile * BK];  // X tile [128][64], three stages (48 KiB)
  __shared__ float red[8][kRowsPerTile];          // per-wave row statistics

  const int b = xcd_remap(blockIdx.x, gridDim.x);
  const int g = find_group(tile_ptr, G, b);
  const int cbeg = chunk_ptr[g];
  const int C = chunk_ptr[g + 1] - cbeg;
  const int rbeg = row_ptr[g], rend = row_ptr[g + 1];
  // Logical order inside a library: groups of kChunkGroup chunks; within a group, row tile major.
  const int RTn = (rend - rbeg + kRowsPerTile - 1) / kRowsPerTile;
  const int local = b - tile_ptr[g];
  const int cg = local / (RTn * kChunkGroup);
  const int gsz = min(kChunkGroup, C - cg * kChunkGroup);
  const int off = local - cg * RTn * kChunkGroup;
  const int rt = off / gsz;
  const int c = cg * kChunkGroup + off % gsz;
  const int row0 = rbeg + rt * kRowsPerTile;
  const int gc = cbeg + c;
  const int nv = min(chunk_nvalid[gc], N);
  const _Float16* Ka = pages_a + (long long)chunk_page[gc] * page_stride;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5;   // lane half: k-group of the fragments, +4 row offset of D
  // Waves 0-3 issue at priority 1, waves 4-7 at 0.  With the waves placed on the SIMDs in turn,
  // waves w and w + 4 share one, and the two, otherwise identical, fall out of step inside a
  // k-step, so one's tail (waits, the next step's first fragments, the barrier) overlaps the
  // other's MFMAs (~0.4 % faster than equal priority, three alternating runs; raising only the
  // k-step body, as the readout does, changed nothing here: both waves of a SIMD meet at the
  // same barrier every k-step).
  if (wv < 4) __builtin_amdgcn_s_setprio(1);
  const int l32 = lane & 31;

  // A fragments of this wave's two slot groups (groups past N/32 re-read the last one; those
  // slots are masked in the epilogue).  Block (sg, kb) starts at ((sg * d/16 + kb) * 64) * 8.
  const _Float16* abase[2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
    abase[mt] = Ka + (long long)min(wv * 2 + mt, N / 32 - 1) * (d / 16) * 512 + lane * 8;
  // B staging, straight from global memory into LDS (gfx950 global_load_lds_dwordx4): a stage is
  // 128 rows x 8 chunks of 16 bytes, LDS chunk id = tid + 512 i (two per thread), and a wave's 64
  // lanes fill 1 KiB of LDS in lane order.  The swizzle is applied on the global side: the lane
  // that fills LDS position p of row r loads the row's chunk p ^ swizzle(r).  Rows past the
  // library re-read its last row (their scores are never stored).
  const _Float16* xdir[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int id = tid + 512 * i;
    const int r = id >> 3;
    xdir[i] = X + (long long)min(row0 + r, rend - 1) * d + (((id & 7) ^ ((r ^ (r >> 3)) & 7)) << 3);
  }
  half8_t fa[2][4];  // [mt][k16 step]: refilled for the next k-step as soon as it is consumed
  auto stage_b = [&](int st, int k0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) stage_to_lds(&lB[st][(512 * i + 64 * wv) * 8], xdir[i] + k0);
  };

  f32x16 acc[2][4];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = (f32x16){};
  // One k-step on LDS stage st.  The scheduling barriers keep every global load where it is
  // written: the compiler otherwise sinks them next to their first use and each k-step waits
  // out a full memory latency.
  // fb0: the first k16 step's B fragments of the coming k-step, read from LDS before the barrier
  // that ends the previous k-step, so the MFMAs start as soon as the barrier releases.
  half8_t fb0[4];
  auto read_fb0 = [&](int st) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
      fb0[nt] = *reinterpret_cast<const half8_t*>(&lB[st][swz(nt * 32 + l32, hl)]);
  };
  // One k-step: four k16 steps of 8 MFMAs.  The B fragments of k16 step ks + 1 are read from
  // LDS while the MFMAs of step ks issue (MFMA and ds_read alternating), and the two A fragment
  // refills go out between the last MFMAs, so no MFMA waits on a read issued just before it.
  // The group barriers fix that order; left alone, the compiler sinks every read to just before
  // its first use.
  auto compute = [&](int st, int knext) {
    half8_t fbn[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      half8_t fb[4];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) fb[nt] = ks == 0 ? fb0[nt] : fbn[nt];
      if (ks < 3)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
          fbn[nt] = *reinterpret_cast<const half8_t*>(&lB[st][swz(nt * 32 + l32, (ks + 1) * 2 + hl)]);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = mfma32(fa[mt][ks], fb[nt], acc[mt][nt]);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
        fa[mt][ks] = *reinterpret_cast<const half8_t*>(abase[mt] + (knext / 16 + ks) * 512);
      if (ks < 3) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
        }
      } else {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 4, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // The prefetch past the last k-step re-reads it (no branch around a load).  The first A
  // fragments load in the loop's own order (k16 step major), so the wait counts the compiler
  // derives for the loop hold on entry too.
  const int nk = d / BK;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) fa[mt][ks] = *reinterpret_cast<const half8_t*>(abase[mt] + ks * 512);
  // Three LDS stages: k-step k reads stage k % 3; at its start it stages the rows of step k + 2
  // into stage (k + 2) % 3 (last read in step k - 1, before the barrier that ended it), waits for
  // them at its end, and reads the first fragments of step k + 1 from stage (k + 1) % 3 (staged in
  // step k - 1 and published by that barrier).  One barrier per k-step.  The staging loads are
  // invisible to the compiler's wait counts, so their waits are explicit: at the end of a
  // k-step only its 8 A fragment refills (issued after the staging) may still be in flight.
  stage_b(0, 0);
  stage_b(1, min(1, nk - 1) * BK);
  wait_vmem<0>();
  __syncthreads();
  read_fb0(0);
  for (int k = 0; k < nk; ++k) {
    const int k1 = min(k + 1, nk - 1) * BK;
    stage_b((k + 2) % 3, min(k + 2, nk - 1) * BK);
    __builtin_amdgcn_sched_barrier(0);
    compute(k % 3, k1);
    wait_vmem<8>();
    read_fb0((k + 1) % 3);
    __syncthreads();
  }
  wait_vmem<0>();

  // acc[mt][nt][r] = S^T[slot][row]: slot = 64w + 32mt + 8(r/4) + 4hl + r%4, row = 32nt + l32.
  auto slot_of = [&](int mt, int r) { return wv * 64 + mt * 32 + (r >> 2) * 8 + hl * 4 + (r & 3); };
  // Octet-major element (row t, slot s of chunk c): ((c*N/8 + s/8) * p_rows + t) * 8 + s%8.
  auto poff = [&](int t, int s0) {
    return ((long long)(c * (N / 8) + (s0 >> 3)) * p_rows + t) * 8 + (s0 & 7);
  };

  if (MODE == 2) {
    // ---- linear read: p = S / sqrt(n_valid), masked slots 0
    const float inv = 1.f / sqrtf((float)nv);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int t = row0 + nt * 32 + l32;
      if (t >= rend) continue;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int s0 = slot_of(mt, q4 * 4);
          if (s0 < N) {
            half4_t h;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              h[e] = (_Float16)(s0 + e < nv ? acc[mt][nt][q4 * 4 + e] * inv : 0.f);
            __builtin_nontemporal_store(h, reinterpret_cast<half4_t*>(P + poff(t, s0)));
          }
        }
    }
  } else if (MODE == 0) {
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
      rmax[nt] = fmaxf(m, swap_partner<32>(m, hl != 0));
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
      rsum[nt] = s + swap_partner<32>(s, hl != 0);
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
      // Optional: the log-sum-exp of the row's scaled scores over the chunk's valid slots
      // (natural log; rmax and s are in log2 units).
      const int t = row0 + nt * 32 + l32;
      if (gamma && wv == 0 && hl == 0 && t < rend)
        gamma[(long long)t * ldg + c] = (rmax[nt] + __log2f(s)) * kLn2;
    }
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int t = row0 + nt * 32 + l32;
      if (t >= rend) continue;
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
            __builtin_nontemporal_store(h, reinterpret_cast<half4_t*>(P + poff(t, s0)));
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
      float s = 0.f;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int s0 = slot_of(mt, q4 * 4);
          pv[mt][nt][q4] = s0 < N ? __builtin_nontemporal_load(reinterpret_cast<const half4_t*>(P + poff(t, s0))) : (half4_t){};
#pragma unroll
          for (int e = 0; e < 4; ++e) s += (float)pv[mt][nt][q4][e] * acc[mt][nt][q4 * 4 + e];
        }
      gpart[nt] = s + swap_partner<32>(s, hl != 0);
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
      const int t = row0 + nt * 32 + l32;
      if (t >= rend) continue;
      if (wv == 0 && hl == 0) gamma[(long long)t * ldg + c] = s;
      const float coef = (MODE == 1 ? temp : 1.f / sqrtf((float)nv)) * w[(long long)t * ldw + c];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int s0 = slot_of(mt, q4 * 4);
          if (s0 < N) {
            half4_t h;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float u = acc[mt][nt][q4 * 4 + e];
              h[e] = (_Float16)(MODE == 1 ? coef * (float)pv[mt][nt][q4][e] * (u - s)
                                          : (s0 + e < nv ? coef * u : 0.f));
            }
            __builtin_nontemporal_store(h, reinterpret_cast<half4_t*>(dS + poff(t, s0)));
          }
        }
    }
  }
}

// ------------------------------------------------------------------------------------------
// Readout kernel: out[t, :] = sum_c scale(t,c) sum_n A[t, c, n] K_c[n, :] (A octet-major).
// Workgroup tile 128 rows x 256 dims, 4 waves; wave w owns dims [64w, 64w+64) x all 128 rows
// (4 x 2 MFMA 32x32 tiles).  The dims of a wave are private to it: their fragments come from the
// layout-B page copy (coalesced 1 KiB loads), refilled for the next k-step as they are consumed;
// the 128 A rows are shared and staged through LDS (three swizzled stages of 16 KiB).  Two
// workgroups run on each CU.
// scale = w[t, c] when w != nullptr (forward read), else 1 (the backward dS already carries it).
// ROUTE (backward): the accumulators start from the routing term sum_c dl[t, c] S[c, :] over the
// library's chunks (fp32 MFMAs) instead of 0.  Rows of one tile belong to one library.
template <bool ROUTE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void readout_kernel(
    const _Float16* __restrict__ A, long long a_rows, const int* __restrict__ row_ptr,
    const int* __restrict__ tile_ptr, int G, const _Float16* __restrict__ pages_b, int N, int d,
    long long page_stride, const int* __restrict__ chunk_ptr, const int* __restrict__ chunk_page,
    const float* __restrict__ w, long long ldw, const float* __restrict__ dl, long long ldl,
    const float* __restrict__ S, float* __restrict__ out, long long ldo) {
  constexpr int RT = kReadoutRows;
  __shared__ _Float16 lA[3][RT * BK];

  const int b = xcd_remap(blockIdx.x, gridDim.x);
  const int g = find_group(tile_ptr, G, b);
  const int local = b - tile_ptr[g];
  const int ntile_d = (d + 255) / 256;
  const int dt = local % ntile_d;
  const int rt = local / ntile_d;
  const int rbeg = row_ptr[g], rend = row_ptr[g + 1];
  const int row0 = rbeg + rt * RT;
  const int d0 = dt * 256;
  const int cbeg = chunk_ptr[g];
  const int C = chunk_ptr[g + 1] - cbeg;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5;
  const int l32 = lane & 31;

  // A staging: RT rows x 8 octets; thread chunk i covers row (tid % RT), octet (tid/RT + 2i):
  // consecutive lanes read consecutive rows of one octet (contiguous in the octet-major A).  All
  // chunks of a thread share its row, hence one scale per k-step, applied when the chunks are
  // stored to LDS (after the k-step's MFMAs, by which time the loads have landed).
  constexpr int NA = RT * 8 / 256;
  const int arow = tid % RT;
  const long long arow_g = min(row0 + arow, rend - 1);
  int aoct[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) aoct[i] = tid / RT + 2 * i;
  u32x4 ra[NA];
  float wa = 1.f;
  auto load_a = [&](int c, int n0) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const long long oct = (long long)c * (N / 8) + n0 / 8 + aoct[i];
      ra[i] = *reinterpret_cast<const u32x4*>(A + (oct * a_rows + arow_g) * 8);
    }
    if (w) wa = w[arow_g * ldw + c];
  };
  auto store_a = [&](int st) {
    if (w) {
      const _Float16 wh = (_Float16)wa;
      const half8_t sc = {wh, wh, wh, wh, wh, wh, wh, wh};
#pragma unroll
      for (int i = 0; i < NA; ++i)
        ra[i] = __builtin_bit_cast(u32x4, __builtin_bit_cast(half8_t, ra[i]) * sc);
    }
#pragma unroll
    for (int i = 0; i < NA; ++i) *reinterpret_cast<u32x4*>(&lA[st][swz(arow, aoct[i])]) = ra[i];
  };
  // B fragments of this wave's two 32-dim groups (groups past d/32 re-read the last one; those
  // columns are not stored).  Block (db, nb) starts at ((db * N/16 + nb) * 64) * 8.
  int dbk[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) dbk[nt] = min((d0 + wv * 64 + nt * 32) / 32, d / 32 - 1);
  auto kb_base = [&](int c) {
    return pages_b + (long long)chunk_page[cbeg + c] * page_stride + lane * 8;
  };
  half8_t fb[2][4];  // [nt][k16 step]

  f32x16 acc[NA][2];
#pragma unroll
  for (int mt = 0; mt < NA; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = (f32x16){};
  if (ROUTE) {
    // The routing term, k = 2 chunks per v_mfma_f32_32x32x2f32: lane l supplies A[l%32][l/32] =
    // dl[row 32mt + l32][chunk c0 + hl] and B[l/32][l%32] = S[chunk c0 + hl][column], and the
    // result lands in the accumulator layout of the read.  Rows past the library and columns past
    // d read clamped addresses and are never stored; a chunk past C contributes 0.  Addresses are
    // 32-bit lane offsets from the tile's (wave-uniform) bases: one register per load.
    const float* dl_tile = dl + (long long)row0 * ldl;
    const float* s_lib = S + (long long)cbeg * d;
    int dlo[NA], so[2];
#pragma unroll
    for (int mt = 0; mt < NA; ++mt) dlo[mt] = (min(row0 + mt * 32 + l32, rend - 1) - row0) * (int)ldl;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) so[nt] = min(d0 + wv * 64 + nt * 32 + l32, d - 1);
#pragma unroll 4
    for (int c0 = 0; c0 < C; c0 += 2) {
      const int cl = c0 + hl;
      const bool live = cl < C;
      const int cc = live ? cl : C - 1;
      float av[NA], bv[2];
#pragma unroll
      for (int mt = 0; mt < NA; ++mt) av[mt] = live ? dl_tile[dlo[mt] + cc] : 0.f;
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) bv[nt] = live ? s_lib[so[nt] + cc * d] : 0.f;
#pragma unroll
      for (int mt = 0; mt < NA; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[mt], bv[nt], acc[mt][nt], 0, 0, 0);
    }
  }
  // fa0: the first k16 step's A fragments of the coming k-step, read before the barrier that
  // ends the previous k-step (as in the scores kernel).
  half8_t fa0[NA];
  auto read_fa0 = [&](int st) {
#pragma unroll
    for (int mt = 0; mt < NA; ++mt)
      fa0[mt] = *reinterpret_cast<const half8_t*>(&lA[st][swz(mt * 32 + l32, hl)]);
  };
  // As in the scores kernel: the A fragments of k16 step ks + 1 are read while the MFMAs of
  // step ks issue, the B refills go out between the last MFMAs, and the body runs at issue
  // priority 1, the tail (the staging stores, the next step's first fragments, the barrier) at 0:
  // the CU's two workgroups are in different phases, and the one issuing MFMAs wins the
  // arbitration (forward and backward ~3 % faster than at equal priority).
  auto compute = [&](int st, const _Float16* kbn, int nbn) {
    half8_t fan[NA];
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      half8_t fa[NA];
#pragma unroll
      for (int mt = 0; mt < NA; ++mt) fa[mt] = ks == 0 ? fa0[mt] : fan[mt];
      if (ks < 3)
#pragma unroll
        for (int mt = 0; mt < NA; ++mt)
          fan[mt] = *reinterpret_cast<const half8_t*>(&lA[st][swz(mt * 32 + l32, (ks + 1) * 2 + hl)]);
#pragma unroll
      for (int mt = 0; mt < NA; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = mfma32(fa[mt], fb[nt][ks], acc[mt][nt]);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
        fb[nt][ks] = *reinterpret_cast<const half8_t*>(kbn + ((long long)dbk[nt] * (N / 16) + nbn + ks) * 512);
      static_assert(NA == 4, "the schedule below is written for 8 MFMAs per k16 step");
      if (ks < 3) {
#pragma unroll
        for (int i = 0; i < NA; ++i) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
        }
      } else {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 4, 0);
      }
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  const int kpc = N / BK;  // k-steps per chunk
  const int total = C * kpc;
  {  // in the loop's own order (k16 step major), as in the scores kernel
    const _Float16* kb0 = kb_base(0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
        fb[nt][ks] = *reinterpret_cast<const half8_t*>(kb0 + ((long long)dbk[nt] * (N / 16) + ks) * 512);
  }
  // Three LDS stages, as in the scores kernel: step it reads stage it % 3, stores the rows of
  // step it + 2 into stage (it + 2) % 3 and reads the first fragments of step it + 1 from stage
  // (it + 1) % 3 before its barrier.
  load_a(0, 0);
  store_a(0);
  {
    const int n1 = min(1, total - 1);
    load_a(n1 / kpc, (n1 % kpc) * BK);
    store_a(1);
  }
  __syncthreads();
  read_fa0(0);
  for (int it = 0; it < total; ++it) {
    const int nx = min(it + 1, total - 1);  // the prefetch past the last step re-reads it
    const int cn = nx / kpc, nn = (nx % kpc) * BK;
    const int n2 = min(it + 2, total - 1);
    load_a(n2 / kpc, (n2 % kpc) * BK);
    __builtin_amdgcn_sched_barrier(0);
    compute(it % 3, kb_base(cn), nn / 16);
    __builtin_amdgcn_s_setprio(0);
    store_a((it + 2) % 3);
    read_fa0((it + 1) % 3);
    __syncthreads();
  }
  // acc[mt][nt][r] = out[row0 + 32mt + 8(r/4) + 4hl + r%4][d0 + 64w + 32nt + l32]
#pragma unroll
  for (int mt = 0; mt < NA; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = row0 + mt * 32 + (r >> 2) * 8 + hl * 4 + (r & 3);
      if (t >= rend) continue;
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int dd = d0 + wv * 64 + nt * 32 + l32;
        if (dd < d) __builtin_nontemporal_store(acc[mt][nt][r], &out[(long long)t * ldo + dd]);
      }
    }
}

// ------------------------------------------------------------------------------------------
// Routing coefficients of the backward: dl[t, c] = route_temp * w (dw - sum_c' w dw) for the
// chunks c of row t's library (dw = dw_read (+ dw_ext when given)); one wave per row.  The
// readout adds sum_c dl[t, c] S[c] to dq.
__global__ __launch_bounds__(256) void route_coef_kernel(
    const float* __restrict__ w, long long ldw, const float* __restrict__ dw_read, long long ldr,
    const float* __restrict__ dw_ext, long long lde, const int* __restrict__ row_ptr, int G,
    const int* __restrict__ chunk_ptr, int M, float route_temp, float* __restrict__ dl,
    long long ldl) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);  // wave-uniform
  const int lane = threadIdx.x & 63;
  if (t >= M) return;
  const int g = find_group(row_ptr, G, t);
  const int C = chunk_ptr[g + 1] - chunk_ptr[g];
  auto dw_of = [&](int c) {
    float dv = dw_read[(long long)t * ldr + c];
    if (dw_ext) dv += dw_ext[(long long)t * lde + c];
    return dv;
  };
  float sdot = 0.f;
  for (int c = lane; c < C; c += 64) sdot += w[(long long)t * ldw + c] * dw_of(c);
  sdot = wave_sum(sdot);
  for (int c = lane; c < C; c += 64)
    dl[(long long)t * ldl + c] = route_temp * w[(long long)t * ldw + c] * (dw_of(c) - sdot);
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
    // Four chunks' S loads in flight per step (the loop otherwise waits out one L2 round trip
    // per chunk).
#pragma unroll 4
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
  const int blocks = std::min(M, 8192);
  hipLaunchKernelGGL(cast_rows_f16_kernel, dim3(blocks), dim3(kCastThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), x, ldx, M, d,
                     static_cast<_Float16*>(y));
  return check_launch();
}

extern "C" int xenc_fragment_pages(const void* pages, long long P, int slots_per_page, int d,
                                   int layout, void* out, void* stream) {
  if (P < 0 || slots_per_page <= 0 || d <= 0 || (layout != 0 && layout != 1)) return XENC_EINVAL;
  if (slots_per_page % 32 != 0 || d % 32 != 0) return XENC_EINVAL;
  if (P == 0) return XENC_OK;
  if (!pages || !out) return XENC_ENULL;
  if (!aligned16(pages) || !aligned16(out)) return XENC_EALIGN;
  const long long total = P * (long long)slots_per_page * d / 8;
  const int blocks = (int)std::min<long long>((total + 255) / 256, 65536);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const _Float16* src = static_cast<const _Float16*>(pages);
  _Float16* dst = static_cast<_Float16*>(out);
  if (layout == 0)
    hipLaunchKernelGGL(fragment_pages_kernel<0>, dim3(blocks), dim3(256), 0, st, src, P,
                       slots_per_page, d, dst);
  else
    hipLaunchKernelGGL(fragment_pages_kernel<1>, dim3(blocks), dim3(256), 0, st, src, P,
                       slots_per_page, d, dst);
  return check_launch();
}

static int check_prefill_common(int d, int N, long long page_stride) {
  if (d <= 0 || d % BK != 0) return XENC_EINVAL;                       // scores k loop
  if (N <= 0 || N > kSlotsPerTile || N % BK != 0) return XENC_EINVAL;  // readout k loop
  if (page_stride < (long long)N * d || page_stride % 8 != 0) return XENC_EINVAL;
  return XENC_OK;
}

extern "C" int xenc_prefill_scores(int mode, const void* x, int d, const int* row_ptr,
                                   const int* tile_ptr, int G, int n_tiles, const void* pages_a,
                                   int slots_per_page, long long page_stride,
                                   const int* chunk_ptr, const int* chunk_page,
                                   const int* chunk_nvalid, float temp, const float* w,
                                   long long ldw, void* p, long long p_rows, void* ds,
                                   float* gamma, long long ldg, void* stream) {
  if (mode < 0 || mode > 3) return XENC_EINVAL;
  if (int rc = check_prefill_common(d, slots_per_page, page_stride)) return rc;
  if (G <= 0 || n_tiles < 0 || p_rows < 0) return XENC_EINVAL;
  if (n_tiles == 0) return XENC_OK;
  if (!x || !row_ptr || !tile_ptr || !pages_a || !chunk_ptr || !chunk_page || !chunk_nvalid || !p)
    return XENC_ENULL;
  const bool bwd = mode & 1;
  if (bwd && (!w || !ds || !gamma)) return XENC_ENULL;
  if (!aligned16(x) || !aligned16(pages_a) || !aligned16(p) || (bwd && !aligned16(ds)))
    return XENC_EALIGN;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const _Float16* X = static_cast<const _Float16*>(x);
  const _Float16* pg = static_cast<const _Float16*>(pages_a);
  auto launch = [&](auto kernel, float t) {
    hipLaunchKernelGGL(kernel, dim3(n_tiles), dim3(512), 0, st, X, d, row_ptr, tile_ptr, G, pg,
                       slots_per_page, page_stride, chunk_ptr, chunk_page, chunk_nvalid, t, w, ldw,
                       static_cast<_Float16*>(p), p_rows, static_cast<_Float16*>(ds), gamma, ldg);
  };
  switch (mode) {
    case 0: launch(scores_kernel<0>, temp * kLog2e); break;
    case 1: launch(scores_kernel<1>, temp); break;
    case 2: launch(scores_kernel<2>, temp); break;
    default: launch(scores_kernel<3>, temp); break;
  }
  return check_launch();
}

extern "C" int xenc_prefill_readout(const void* a, long long a_rows, const int* row_ptr,
                                    const int* tile_ptr, int G, int n_tiles, const void* pages_b,
                                    int slots_per_page, int d, long long page_stride,
                                    const int* chunk_ptr, const int* chunk_page, const float* w,
                                    long long ldw, float* out, long long ldo, void* stream) {
  if (int rc = check_prefill_common(d, slots_per_page, page_stride)) return rc;
  if (G <= 0 || n_tiles < 0 || a_rows < 0 || ldo < d) return XENC_EINVAL;
  if (n_tiles == 0) return XENC_OK;
  if (!a || !row_ptr || !tile_ptr || !pages_b || !chunk_ptr || !chunk_page || !out)
    return XENC_ENULL;
  if (!aligned16(a) || !aligned16(pages_b)) return XENC_EALIGN;
  hipLaunchKernelGGL(readout_kernel<false>, dim3(n_tiles), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const _Float16*>(a), a_rows,
                     row_ptr, tile_ptr, G, static_cast<const _Float16*>(pages_b), slots_per_page,
                     d, page_stride, chunk_ptr, chunk_page, w, ldw, nullptr, 0, nullptr, out, ldo);
  return check_launch();
}

extern "C" int xenc_prefill_readout_routed(const void* ds, long long a_rows, const int* row_ptr,
                                           const int* tile_ptr, int G, int n_tiles,
                                           const void* pages_b, int slots_per_page, int d,
                                           long long page_stride, const int* chunk_ptr,
                                           const int* chunk_page, const float* w, long long ldw,
                                           const float* dw_read, long long ldr,
                                           const float* dw_ext, long long lde, const float* S,
                                           int cmax, float route_temp, float* dl, long long ldl,
                                           float* dq, long long ldq, void* stream) {
  if (int rc = check_prefill_common(d, slots_per_page, page_stride)) return rc;
  if (G <= 0 || n_tiles < 0 || a_rows < 0 || a_rows > INT_MAX || cmax <= 0 || ldq < d ||
      ldl < cmax || ldw < cmax || ldr < cmax || (dw_ext && lde < cmax))
    return XENC_EINVAL;
  // 32-bit offsets inside a readout tile (128 rows of dl) and a library's summaries (cmax rows of S)
  if ((long long)kReadoutRows * ldl > INT_MAX || (long long)cmax * d > INT_MAX) return XENC_EINVAL;
  if (n_tiles == 0 || a_rows == 0) return XENC_OK;
  if (!ds || !row_ptr || !tile_ptr || !pages_b || !chunk_ptr || !chunk_page || !w || !dw_read ||
      !S || !dl || !dq)
    return XENC_ENULL;
  if (!aligned16(ds) || !aligned16(pages_b)) return XENC_EALIGN;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int M = (int)a_rows;
  hipLaunchKernelGGL(route_coef_kernel, dim3((M + 3) / 4), dim3(256), 0, st, w, ldw, dw_read,
                     ldr, dw_ext, lde, row_ptr, G, chunk_ptr, M, route_temp, dl, ldl);
  if (int rc = check_launch()) return rc;
  hipLaunchKernelGGL(readout_kernel<true>, dim3(n_tiles), dim3(256), 0, st,
                     static_cast<const _Float16*>(ds), a_rows, row_ptr, tile_ptr, G,
                     static_cast<const _Float16*>(pages_b), slots_per_page, d, page_stride,
                     chunk_ptr, chunk_page, nullptr, 0, dl, ldl, S, dq, ldq);
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
