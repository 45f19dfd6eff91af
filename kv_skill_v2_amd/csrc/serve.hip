// Serving-side decode step of op B, on the device: the per-step block tables and lengths of the
// joint decode read, and the writes of the step's own K/V rows into the paged own-row pool.
//
// The reference rebuilds the per-row metadata on the host every decode step and copies it to
// the device (Static.fill, xenc/d23_vllm_plugin.py:433-457; positions tracked by stage_step,
// :241-264), then writes the new own rows with index_copy_ (read_static, :486-487).  Here the
// per-request state lives on the device and one kernel advances it, so a decode step (advance,
// own-row write, joint read) can be captured once and replayed step after step; the host only
// touches the state when a request is admitted or leaves.
//
// Request slot s (int32 x 4): {op_start block, op_tokens, own_len, unused}.  Slot s owns blocks
// [s * own_blocks, (s + 1) * own_blocks) of the own pool.  Row i of a step decodes one token of
// slot row_slot[i] (< 0: a padded row).  A slot appears in at most one row of a step.
#include "xenc_common.h"

namespace xenc {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void decode_step_kernel(
    [[maybe_unused]] int N, const int* __restrict__ row_slot, int* __restrict__ slots, int n_slots, int own_blocks,
    int block_size, int max_op_blocks, int dummy_block, int* __restrict__ op_bt, long long ld_op,
    int* __restrict__ op_len, int* __restrict__ own_bt, long long ld_own, int* __restrict__ own_len,
    long long* __restrict__ write_pos) {
  const int i = blockIdx.x;
  const int s = row_slot[i];
  const bool live = s >= 0 && s < n_slots;
  int op_start = 0, op_tok = 0;
  if (live) {
    op_start = slots[s * 4 + 0];
    op_tok = slots[s * 4 + 1];
  }
  const int op_blk = (op_tok + block_size - 1) / block_size;
  for (int j = threadIdx.x; j < max_op_blocks; j += blockDim.x)
    op_bt[i * ld_op + j] = (live && j < op_blk) ? op_start + j : dummy_block;
  for (int j = threadIdx.x; j < own_blocks; j += blockDim.x)
    own_bt[i * ld_own + j] = live ? s * own_blocks + j : 0;
  if (threadIdx.x == 0) {
    op_len[i] = op_tok;
    if (!live) {
      own_len[i] = 0;
      write_pos[i] = -1;
    } else {
      const int p0 = slots[s * 4 + 2];
      const int cap = own_blocks * block_size;
      if (p0 < cap) {  // the new token's own row goes at position p0
        write_pos[i] = (long long)s * cap + p0;
        own_len[i] = p0 + 1;
        slots[s * 4 + 2] = p0 + 1;
      } else {         // own rows full: read without writing (the caller sizes own_blocks)
        write_pos[i] = -1;
        own_len[i] = cap;
      }
    }
  }
}

// Own pool [num_blocks, block_size, hkv, d] (element strides sb, ss, sh; d contiguous); the new
// rows k_new / v_new [N, hkv, d] (strides s_n, s_h).  Row i goes to pool row write_pos[i]
// (block write_pos / block_size, slot write_pos % block_size); rows with write_pos < 0 are
// skipped.  16-byte copies, 2-byte elements (fp16 / bf16 alike).
__global__ __launch_bounds__(256) void own_rows_write_kernel(
    int hkv, int d, const unsigned short* __restrict__ k_new, const unsigned short* __restrict__ v_new,
    long long s_n, long long s_h, unsigned short* __restrict__ own_k, unsigned short* __restrict__ own_v,
    long long sb, long long ss, long long sh, int block_size, const long long* __restrict__ write_pos) {
  const int i = blockIdx.x;
  const long long p = write_pos[i];
  if (p < 0) return;
  const long long blk = p / block_size, slot = p % block_size;
  const int per_head = d / 8;
  for (int t = threadIdx.x; t < hkv * per_head; t += blockDim.x) {
    const int h = t / per_head, c = (t % per_head) * 8;
    const long long src = i * s_n + h * s_h + c;
    const long long dst = blk * sb + slot * ss + h * sh + c;
    *reinterpret_cast<u32x4*>(own_k + dst) = *reinterpret_cast<const u32x4*>(k_new + src);
    *reinterpret_cast<u32x4*>(own_v + dst) = *reinterpret_cast<const u32x4*>(v_new + src);
  }
}

}  // namespace
}  // namespace xenc

using namespace xenc;

extern "C" int xenc_decode_step(int N, const int* row_slot, int* slots, int n_slots, int own_blocks,
                                int block_size, int max_op_blocks, int dummy_block, int* op_bt,
                                long long ld_op_bt, int* op_len, int* own_bt, long long ld_own_bt,
                                int* own_len, long long* write_pos, void* stream) {
  if (N < 0 || n_slots <= 0 || own_blocks <= 0 || block_size <= 0 || max_op_blocks <= 0 ||
      dummy_block < 0 || ld_op_bt < max_op_blocks || ld_own_bt < own_blocks)
    return XENC_EINVAL;
  if ((long long)n_slots * own_blocks * block_size > 0x7fffffffLL) return XENC_EINVAL;
  if (N == 0) return XENC_OK;
  if (!row_slot || !slots || !op_bt || !op_len || !own_bt || !own_len || !write_pos) return XENC_ENULL;
  hipLaunchKernelGGL(decode_step_kernel, dim3(N), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     N, row_slot, slots, n_slots, own_blocks, block_size, max_op_blocks, dummy_block,
                     op_bt, ld_op_bt, op_len, own_bt, ld_own_bt, own_len, write_pos);
  return check_launch();
}

extern "C" int xenc_own_rows_write(int N, int hkv, int d, const void* k_new, const void* v_new,
                                   long long s_n, long long s_h, void* own_k, void* own_v,
                                   long long sb, long long ss, long long sh, int block_size,
                                   const long long* write_pos, void* stream) {
  if (N < 0 || hkv <= 0 || d <= 0 || d % 8 != 0 || block_size <= 0) return XENC_EINVAL;
  if (s_n % 8 != 0 || s_h % 8 != 0 || sb % 8 != 0 || ss % 8 != 0 || sh % 8 != 0) return XENC_EALIGN;
  if (N == 0) return XENC_OK;
  if (!k_new || !v_new || !own_k || !own_v || !write_pos) return XENC_ENULL;
  if (!aligned16(k_new) || !aligned16(v_new) || !aligned16(own_k) || !aligned16(own_v))
    return XENC_EALIGN;
  hipLaunchKernelGGL(own_rows_write_kernel, dim3(N), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), hkv, d,
                     static_cast<const unsigned short*>(k_new), static_cast<const unsigned short*>(v_new),
                     s_n, s_h, static_cast<unsigned short*>(own_k), static_cast<unsigned short*>(own_v),
                     sb, ss, sh, block_size, write_pos);
  return check_launch();
}
