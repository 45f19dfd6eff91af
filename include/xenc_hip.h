/*
 * xenc_hip.h — C ABI of the MI355X Library-read library (libxenc_hip.so).
 *
 * Every entry point takes device pointers, element strides and sizes, plus an opaque
 * `stream` (a hipStream_t; NULL = the null stream).  No entry point allocates device or host
 * memory, synchronises the stream or reads device memory on the host, so every call can be
 * captured into a HIP graph.  Work buffers are passed in by the caller; their sizes come from
 * the *_workspace_bytes queries.  Return value: XENC_OK (0) or a negative XENC_E* code;
 * xenc_strerror() names it and xenc_last_hip_error() gives the HIP error of a failed launch.
 *
 * Data layout shared by the Library-read entry points ("library set"):
 *   pages        fp16 [P, slots_per_page, d]  chunk operators, one chunk per page, slot rows
 *                contiguous (d fastest); K = V (tied): the same rows are keys and values.
 *   chunk_ptr    int32 [G+1]    chunks of library g are global chunks chunk_ptr[g] .. chunk_ptr[g+1]-1
 *   chunk_page   int32 [Ctot]   page holding global chunk c (any order: the page table)
 *   chunk_nvalid int32 [Ctot]   valid slots of chunk c (1 .. slots_per_page); rows past it are masked
 *   S            fp32  [Ctot, d] summary key of chunk c (L2-normalised masked mean of its slots)
 *   q            fp32  [M, ldq]  query rows (already L2-normalised by the caller)
 *   q_group      int32 [M]       library read by query row m
 * Routed chunk indices are LOCAL to the query's library (0 .. C_g-1), as the reference's
 * per-library top-k returns them.
 */
#ifndef XENC_HIP_H
#define XENC_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  XENC_OK = 0,
  XENC_EINVAL = -1,      /* a size/argument is out of range (d % 8 != 0, k < 0, M < 0 ...) */
  XENC_ENULL = -2,       /* a required pointer is NULL */
  XENC_EALIGN = -3,      /* a pointer or stride breaks the 16-byte alignment the kernels need */
  XENC_EWORKSPACE = -4,  /* the workspace passed in is smaller than the size query returned */
  XENC_EHIP = -5,        /* a kernel launch failed; see xenc_last_hip_error() */
  XENC_ESCRATCH = -6     /* the call needs more than the allocation-free entry point's fixed scratch */
};

const char* xenc_strerror(int code);
int xenc_last_hip_error(void);
/* ABI version: bumped whenever a signature or a calling contract below changes. */
int xenc_abi_version(void);

/*
 * Routing: logit[m,c] = route_temp * <q[m], S[chunk_ptr[g]+c]>, g = q_group[m].
 * If 0 < top_k < C_g keep the top_k largest (ties -> lower chunk index), else keep all C_g.
 * w = softmax over the kept logits (the others are -inf, i.e. weight 0).
 * Outputs: w_dense [M, ldw] (columns >= C_g are 0; max C_g <= ldw <= 5460),
 *          idx [M, kk] int32 kept chunks, -1 past the kept count: in descending-logit order
 *          (ties -> lower index) under top-k, in chunk order 0..C_g-1 when all are kept,
 *          w_sel [M, kk] their weights (0 past the kept count).
 * kk must be >= min(top_k, C_g) for top-k and >= C_g for dense routing.
 * Replaces LibraryInjector.route (xenc/injector.py:220-229).
 */
int xenc_route_topk(const float* q, long long ldq, int M, int d,
                    const float* S, const int* chunk_ptr, const int* q_group, int G,
                    int top_k, float route_temp,
                    float* w_dense, long long ldw, int* idx, float* w_sel, int kk,
                    void* stream);

/*
 * Routing of many query rows grouped by library (prefill / registration): rows of library g are
 * row_ptr[g] .. row_ptr[g+1]-1; tile_ptr[g] = sum_{g'<g} ceil(T_g'/32) * ceil(C_g'/32) (G+1
 * entries, n_tiles = tile_ptr[G]).  Same outputs and top-k / softmax as xenc_route_topk; the dots
 * are computed as 32-row x 32-chunk fp32 tiles (each summary row read once per 32 query rows).
 * ldw <= 1364.  q_f16 (optional, 16-byte aligned): also writes q as contiguous fp16 rows
 * [M, d] (the operand of xenc_prefill_scores), from the same read of q.
 * Replaces LibraryInjector.route (xenc/injector.py:220-229) for many tokens.
 */
int xenc_route_topk_rows(const float* q, long long ldq, int M, int d, const float* S,
                         const int* chunk_ptr, const int* row_ptr, const int* tile_ptr, int G,
                         int n_tiles, int top_k, float route_temp, float* w_dense, long long ldw,
                         int* idx, float* w_sel, int kk, void* q_f16, void* stream);

/*
 * Decode read over routed pages (split-K over slots, log-sum-exp merge):
 *   softmax=1: r[m] = sum_j w_sel[m,j] * sum_n softmax_n(read_temp*<q,K[c_j,n]>) K[c_j,n]
 *   softmax=0: r[m] = sum_j w_sel[m,j] * sum_n <q,K[c_j,n]>/sqrt(n_valid) K[c_j,n]  (linear read)
 * over the valid slots n of the routed chunks c_j = idx[m,j] (entries < 0 are skipped).
 * Each slot row is read from HBM once for both the score and the value.  Page slots are
 * split into nsplit ranges of ceil(slots_per_page/nsplit) slots (nsplit in 1..64).
 * r is fp32 [M, ldr].  The partials of a query are merged in a fixed order by a second kernel
 * of the same call, so results are deterministic.
 * Workspace: xenc_decode_workspace_bytes(max_rows, kk, nsplit, d) bytes for calls of up to
 * max_rows query rows (pass the same max_rows to every call); set it up once with
 * xenc_decode_workspace_init (a kernel, no memset), then reuse it for calls of any
 * M <= max_rows.  Calls that share a workspace must not overlap (same stream, or ordered).
 * Replaces the read of LibraryInjector._branch (xenc/injector.py:236-265) when the routed
 * chunks are known: equal to reading every chunk with w = 0 off the top-k.
 */
size_t xenc_decode_workspace_bytes(int max_rows, int kk, int nsplit, int d);
int xenc_decode_workspace_init(void* workspace, size_t workspace_bytes, int max_rows, void* stream);
int xenc_library_read_decode(const float* q, long long ldq, int M, int d,
                             const void* pages, int slots_per_page, long long page_stride,
                             const int* chunk_page, const int* chunk_nvalid,
                             const int* chunk_ptr, const int* q_group, int G,
                             const int* idx, const float* w_sel, int kk,
                             float read_temp, int softmax, int nsplit,
                             float* r, long long ldr,
                             void* workspace, size_t workspace_bytes, int max_rows, void* stream);

/*
 * Routing and the decode read in one call: xenc_route_topk's outputs (w_dense, idx, w_sel) and
 * xenc_library_read_decode's r, same arguments as the two calls together, same results bit for
 * bit.  When every library has at most 64 chunks (ldw <= 64) and the rows do not share libraries
 * (the page-grouped order needs the routed chunks first), the top-k + softmax runs in the read
 * kernel's prologue instead of a kernel of its own: the q . S dots go to the workspace first (for
 * libraries of at most 16 chunks, ldw <= 16, the read workgroups form them too, with no launch of
 * their own), each read workgroup ranks its row's dots itself, and the workgroup of the row's
 * first routed slot writes the dense weights.  Otherwise it makes the two calls.  Workspace as for
 * xenc_library_read_decode.
 * Replaces LibraryInjector.route and the read of _branch (xenc/injector.py:220-265) for decode rows.
 */
int xenc_route_read_decode(const float* q, long long ldq, int M, int d, const float* S,
                           const void* pages, int slots_per_page, long long page_stride,
                           const int* chunk_page, const int* chunk_nvalid, const int* chunk_ptr,
                           const int* q_group, int G, int top_k, float route_temp,
                           float* w_dense, long long ldw, int* idx, float* w_sel, int kk,
                           float read_temp, int softmax, int nsplit, float* r, long long ldr,
                           void* workspace, size_t workspace_bytes, int max_rows, void* stream);

/*
 * Allocation-free variant of xenc_library_read_decode: the same read, the same arguments without
 * the workspace.  Its partials and page order live in a file-scope device array
 * of XENC_DECODE_SCRATCH_BYTES bytes (64 MiB) that each GPU the library runs on holds until the
 * process ends; calls of up to XENC_DECODE_SCRATCH_ROWS query rows whose workspace
 * (xenc_decode_workspace_bytes(XENC_DECODE_SCRATCH_ROWS, kk, nsplit, d) for those rows) fits in
 * it are accepted, larger ones return XENC_ESCRATCH.  No hipMalloc, hipFree or allocating
 * library call is made.  The first call on a device (with that device current) looks the array
 * up and sets it up with a kernel; make it before capturing a graph.  Every call on one
 * GPU shares that GPU's array: calls that overlap on one GPU (different streams, not ordered)
 * race and give wrong results.
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 */
#define XENC_DECODE_SCRATCH_BYTES (64u << 20)
#define XENC_DECODE_SCRATCH_ROWS 1024
int xenc_library_read_decode_noalloc(const float* q, long long ldq, int M, int d,
                                     const void* pages, int slots_per_page, long long page_stride,
                                     const int* chunk_page, const int* chunk_nvalid,
                                     const int* chunk_ptr, const int* q_group, int G,
                                     const int* idx, const float* w_sel, int kk,
                                     float read_temp, int softmax, int nsplit,
                                     float* r, long long ldr, void* stream);

/*
 * ---- Prefill / registration read (many query rows per library; MFMA, fp16 in, fp32 accumulate)
 * Query rows are grouped by library: rows of library g are row_ptr[g] .. row_ptr[g+1]-1.
 * Tiles: the scores kernel takes tile_ptr[g] = sum_{g'<g} ceil(T_g'/128) * C_g' (G+1 entries,
 * n_tiles = tile_ptr[G]); the readout kernel takes tile_ptr[g] = sum ceil(T_g'/128) * ceil(d/256);
 * the route backward takes tile_ptr[g] = sum ceil(T_g'/16).  Requirements: d % 64 == 0,
 * slots_per_page % 64 == 0 and <= 512.  The probability rows p / dS are fp16 and octet-major:
 * element (row t, chunk c of the row's library, slot n) sits at ((c*slots/8 + n/8)*p_rows + t)*8 + n%8
 * (p_rows >= M; the buffer holds max_C * slots * p_rows halves).
 * The kernels read the pages through two fragment-ordered copies built once per pool by
 * xenc_fragment_pages: layout 0 (scores) is [P][slots/32][d/16][64][8] with lane l of block
 * (sg, kb) = K[32sg + l%32][16kb + 8(l/32) + e]; layout 1 (readout) is [P][d/32][slots/16][64][8]
 * with lane l of block (db, nb) = K[16nb + 8(l/32) + e][32db + l%32].  page_stride is the stride
 * of one page in the copy (>= slots*d).
 *
 * xenc_prefill_scores(mode=0): p = masked softmax_n(temp * <x_t, K[c,n]>) per (row, chunk); when
 *     gamma is not NULL also gamma[t, c] = logsumexp_n(temp * <x_t, K[c,n]>) over the valid slots
 *     (the per-chunk normaliser, used to join sub-pages of a page longer than 512 slots).
 * xenc_prefill_scores(mode=1): x = upstream gradient g; u = <g_t, K[c,n]>;
 *     gamma[t,c] = sum_n p u  (= dL/dw[t,c] through the read) and
 *     ds[t, c, n] = temp * w[t,c] * p * (u - gamma[t,c]).
 * xenc_prefill_readout: out[t] = sum_c scale(t,c) sum_n a[t, c, n] K[c, n], scale = w[t,c] when w
 *     is given (forward read) else 1 (backward: out = dq through the read).
 * xenc_route_backward: dq[t] += route_temp * sum_c w (dw - sum_c' w dw) S[c],
 *     dw = dw_read (+ dw_ext when not NULL): the gradient through routing.
 * xenc_prefill_readout_routed: the backward's readout with the routing term folded in (its
 *     accumulators start from it):
 *     dq[t] = sum_{c,n} ds[t, c, n] K[c, n] + sum_c dl[t, c] S[c], where
 *     dl[t, c] = route_temp * w (dw - sum_c' w dw) (dw = dw_read (+ dw_ext)) is first written to
 *     the caller's dl [a_rows, ldl >= cmax] fp32 buffer.  dq is written, not accumulated: one
 *     pass over dq where xenc_prefill_readout + xenc_route_backward take three.
 * Replace the forward and the autograd backward of LibraryInjector.route + _branch
 * (xenc/injector.py:220-265) for registration (scripts/register_doc.py:699).
 */
int xenc_cast_rows_f16(const float* x, long long ldx, int M, int d, void* y, void* stream);
int xenc_fragment_pages(const void* pages, long long P, int slots_per_page, int d, int layout,
                        void* out, void* stream);
int xenc_prefill_scores(int mode, const void* x, int d, const int* row_ptr, const int* tile_ptr,
                        int G, int n_tiles, const void* pages_a, int slots_per_page,
                        long long page_stride, const int* chunk_ptr, const int* chunk_page,
                        const int* chunk_nvalid, float temp, const float* w, long long ldw,
                        void* p, long long p_rows, void* ds, float* gamma, long long ldg,
                        void* stream);
int xenc_prefill_readout(const void* a, long long a_rows, const int* row_ptr, const int* tile_ptr,
                         int G, int n_tiles, const void* pages_b, int slots_per_page, int d,
                         long long page_stride, const int* chunk_ptr, const int* chunk_page,
                         const float* w, long long ldw, float* out, long long ldo, void* stream);
int xenc_route_backward(const float* w, long long ldw, const float* dw_read, long long ldr,
                        const float* dw_ext, long long lde, const int* row_ptr,
                        const int* tile_ptr, int G, int n_tiles, int cmax, const float* S,
                        const int* chunk_ptr, int d, float route_temp, float* dq, long long ldq,
                        void* stream);
int xenc_prefill_readout_routed(const void* ds, long long a_rows, const int* row_ptr,
                                const int* tile_ptr, int G, int n_tiles, const void* pages_b,
                                int slots_per_page, int d, long long page_stride,
                                const int* chunk_ptr, const int* chunk_page, const float* w,
                                long long ldw, const float* dw_read, long long ldr,
                                const float* dw_ext, long long lde, const float* S, int cmax,
                                float route_temp, float* dl, long long ldl, float* dq,
                                long long ldq, void* stream);

/*
 * ---- Write-back through the interface's B (decode path)
 *   out[m, o] = row_scale[m] * (sum_k W_g[o, k] r[m, k] + bias_g[o]),  g = row_group[m]
 * r fp32 [M, ldr] (the read, d columns); W fp32: library g's [d_out, d] weight (out-major rows
 * of ldw floats) at W + g * w_group_stride; bias (optional) fp32 d_out floats at
 * bias + g * bias_group_stride (0 = one bias for all libraries); row_scale (optional) fp32 [M]:
 * gain_scale * exp(log_gain) * gate of each row; row_group (optional, NULL = all rows in
 * library 0) int32 [M], clamped to [0, G).  out fp32 [M, ldo].  M <= 4096, G <= 1024,
 * d % 4 == 0, ldr and ldw multiples of 4, r and W 16-byte aligned.  Each used library's W is
 * streamed from HBM once per call: its rows are taken in batches of 8 whose workgroups read the
 * same W rows side by side on one XCD (the later ones from L2); libraries with no rows are not
 * read.  Deterministic.
 * Replaces itf_write and the delta product of LibraryInjector._branch
 * (xenc/injector.py:71-74, 266-267) on the decode path.
 */
int xenc_write_back(const float* r, long long ldr, int M, int d, const int* row_group, int G,
                    const float* W, long long w_group_stride, long long ldw, int d_out,
                    const float* bias, long long bias_group_stride, const float* row_scale,
                    float* out, long long ldo, void* stream);

/*
 * ---- Library pool build from a document cache
 * rows fp16 [R, d] holds the slot rows of C chunks back to back: chunk c is rows
 * row_off[c] .. row_off[c+1]-1 (int64 [C+1], device).  For each chunk, on fp32 values:
 *   x_n      = row n, or L2(row n - mu) = (row - mu) / (|row - mu| + 1e-6) when mu (fp32 [d]) is given
 *   page c   = x_0 .. x_{n_c-1} then zero rows up to slots_per_page, each zero-padded to d_pad,
 *              stored fp16 at pages + c * page_stride (halves)
 *   S[c]     = m / (|m| + 1e-6), m = sum_n x_n / max(n_c, 1), fp32 at S + c * lds (d_pad floats)
 *   nvalid[c] = n_c
 * The caller guarantees n_c <= slots_per_page (a longer chunk is cut to slots_per_page rows).
 * d % 8 == 0, d <= d_pad <= 4096, d_pad % 8 == 0, page_stride >= slots_per_page * d_pad.
 * Deterministic: the column sums merge in a fixed order.
 * Replaces the padding, centring and summaries of Library.__init__ / _summaries
 * (xenc/library.py:47-74) over the cache that load_doc_cache returns (xenc/depth_skill.py:299-311).
 */
int xenc_build_pages(const void* rows, const long long* row_off, int C, int d, const float* mu,
                     int slots_per_page, int d_pad, void* pages, long long page_stride, float* S,
                     long long lds, int* nvalid, void* stream);

/*
 * ---- Op B: joint decode read over a document operator's pages and the request's own pages
 * For query row n < N and query head hq_i = h*G + g (G = hq / hkv, 1 <= G <= 8):
 *   keys/values = [op pool rows 0..op_len[n]-1 ; own pool rows 0..own_len[n]-1]
 *   out[n, hq_i] = softmax_l(scale * <q[n, hq_i], K_l[h]>) . V_l[h]    (one softmax over both)
 * Row l of a pool is block bt[n, l / block_size], slot l % block_size.  Pools are
 * [num_blocks, block_size, hkv, d] with element strides (sb, ss, sh) and d contiguous; K and V
 * pools of one kind share shape and strides.  dtype: 0 = fp16, 1 = bf16 (q, pools); out fp32
 * [N, hq, d] with strides (s_on, s_oh).  d % 8 == 0, d <= 512, G * d <= 4096; a pool block
 * (sb, block_size * ss) and hkv * sh stay below 2^31 elements (else XENC_EINVAL).  Rows with no keys
 * give 0.  The joined range is split into nsplit ranges of `chunk` keys (the last split also
 * takes any keys past nsplit * chunk).  The caller guarantees op_len[n] <= op_bt row width *
 * block size and that block ids lie in the pool (they are device data; nothing is read back).
 * Workspace: xenc_joint_workspace_bytes(max_n, hkv, nsplit, G, d) bytes, initialised once by
 * xenc_joint_workspace_init (its per-(row, kv head) counters are left zero by every call); each
 * call passes the same max_n and N <= max_n.
 * Replaces DecodeReader.__call__ (xenc/d23_read_kernels.py:134-160; math :31-47) as called by
 * read_static (xenc/d23_vllm_plugin.py:489-491).
 */
size_t xenc_joint_workspace_bytes(int max_n, int hkv, int nsplit, int g, int d);
int xenc_joint_workspace_init(void* workspace, size_t workspace_bytes, int max_n, int hkv,
                              void* stream);
int xenc_paged_decode_joint(int dtype, int N, int hq, int hkv, int d,
                            const void* q, long long s_qn, long long s_qh,
                            const void* op_k, const void* op_v, long long op_sb, long long op_ss,
                            long long op_sh, int op_bs, const int* op_bt, long long op_bt_stride,
                            const int* op_len,
                            const void* own_k, const void* own_v, long long own_sb,
                            long long own_ss, long long own_sh, int own_bs, const int* own_bt,
                            long long own_bt_stride, const int* own_len,
                            float scale, int nsplit, int chunk,
                            float* out, long long s_on, long long s_oh,
                            void* workspace, size_t workspace_bytes, int max_n, void* stream);

/*
 * ---- LayerSelector and the epilogue's row scale
 * xenc_selector_weights: per row b of z fp32 [B, ldz] (n candidates, n <= 256, k <= min(n, 64)):
 *   keep the k largest (descending, ties to the lower index), w = softmax over them, 0 elsewhere;
 *   writes w fp32 [B, ldw] (dense), idx int32 [B, ld_sel] and w_sel fp32 [B, ld_sel] (rank order).
 *   Replaces LayerSelector._weights_from_logits (xenc/selector.py:59-67) without straight-through.
 * xenc_selector_apply: out[b] = sum_{j<k} w_row[b*k+j] * exp(*log_alpha) * delta[b*k+j] / (rel + 1e-6),
 *   rel = |delta[b*k+j]| / (|h[b]| + 1e-6); delta fp32 [B*k, ldd], h fp32 [B, ldh], out [B, ldo],
 *   d columns, k <= 64; log_alpha is a device fp32 scalar (read by the kernel, no host sync).  k = 1 is LayerSelector.apply (xenc/selector.py:106-110); k > 1 sums the k
 *   selected layers' updates of a token.
 * xenc_gate_scale: scale[m] = gain_scale * exp(log_gain[p]) * sigmoid(<hn[t], gate_w> + gate_b[p]),
 *   t = row_token[m] (NULL: m), p = row_pos[m] clamped to [0, n_pos) (NULL: 0); hn fp32 [*, ldh]
 *   with d columns.  The per-row factor of delta (itf_gate, itf_gain, xenc/injector.py:59-69).
 */
int xenc_selector_weights(const float* z, long long ldz, int B, int n, int k, float* w, long long ldw,
                          int* idx, float* w_sel, long long ld_sel, void* stream);
int xenc_selector_apply(int B, int k, int d, const float* delta, long long ldd, const float* h,
                        long long ldh, const float* w_row, const float* log_alpha, float* out,
                        long long ldo, void* stream);
int xenc_gate_scale(int M, int d, const float* hn, long long ldh, const int* row_token,
                    const int* row_pos, int n_pos, const float* gate_w, const float* gate_b,
                    const float* log_gain, float gain_scale, float* scale, void* stream);

/*
 * xenc_multi_depth_prepare: the per-token work of a multi-depth decode step in one launch.  Per
 *   token b < B: xenc_selector_weights on z[b] (n depths, top k) into w / idx / w_sel; for each
 *   kept depth p = idx[b, j]: q_rows[b*k + j] = q_all[p * q_depth_stride + b * q_token_stride ..
 *   + d) (the query row of that depth), and scale[b*k + j] = gain_scale * exp(log_gain[p]) *
 *   sigmoid(<hn[b], gate_w> + gate_b[p]) (xenc_gate_scale with row_token = b, row_pos = p; hn fp32
 *   [B, ldh] with d_r columns; gate_b and log_gain hold n entries).  Every output equals the
 *   separate entry points' bit for bit.  Composes LayerSelector._weights_from_logits
 *   (xenc/selector.py:59-67), the per-layer query of the branch (xenc/injector.py:220-229 run at
 *   each kept layer) and itf_gate / itf_gain (xenc/injector.py:59-69).
 */
int xenc_multi_depth_prepare(const float* z, long long ldz, int B, int n, int k, const float* q_all,
                             long long q_depth_stride, long long q_token_stride, int d, const float* hn,
                             long long ldh, int d_r, const float* gate_w, const float* gate_b,
                             const float* log_gain, float gain_scale, float* w, long long ldw, int* idx,
                             float* w_sel, long long ld_sel, float* q_rows, long long ldr, float* scale,
                             void* stream);

/*
 * xenc_multi_depth_prepare_route: xenc_multi_depth_prepare followed by the routing of the B*k rows
 *   (xenc_route_topk with q = q_rows, q_group = idx, the depth of each row as its library), with
 *   the routing dots computed in the same launch as the per-token work, so the step needs one
 *   launch fewer.  n <= 64 depths and ld_sel == k (idx is then the [B*k] library of each row);
 *   d % 8 == 0, d <= 4096, q_all and S 16-byte aligned with strides that keep every row aligned.
 *   The routing outputs are w_dense [B*k, ldwd] (the dots are formed there, then replaced by the
 *   dense weights), ridx / rw_sel [B*k, kk].  Every output equals xenc_multi_depth_prepare then
 *   xenc_route_topk bit for bit (B*k below 256 rows, where xenc_route_topk takes the same dots
 *   and selection kernels).  Composes xenc/selector.py:59-67 and LibraryInjector.route
 *   (xenc/injector.py:220-229) at each kept layer.
 */
int xenc_multi_depth_prepare_route(const float* z, long long ldz, int B, int n, int k,
                                   const float* q_all, long long q_depth_stride,
                                   long long q_token_stride, int d, const float* hn, long long ldh,
                                   int d_r, const float* gate_w, const float* gate_b,
                                   const float* log_gain, float gain_scale, float* w, long long ldw,
                                   int* idx, float* w_sel, long long ld_sel, float* q_rows,
                                   long long ldr, float* scale, const float* S,
                                   const int* chunk_ptr, int G, int top_k, float route_temp,
                                   float* w_dense, long long ldwd, int* ridx, float* rw_sel, int kk,
                                   void* stream);

/*
 * ---- Slot top-k selection read (D8)
 * xenc_select_scores: scores[b, i] = pool over query heads h of <q[b, h], keys[i, h / G]>
 *   (G = n_q / n_kv; pool_mean = 0: max, 1: mean), -inf where valid[i] == 0 (valid may be NULL).
 *   q fp32 [B, n_q, hd], keys fp32 [S, n_kv, hd], scores fp32 [B, ld_s].
 *   Replaces TopKSelector.head_scores + pool_scores at the last position
 *   (xenc/topk_read.py:205-226).
 * xenc_topk_rows: idx[b, :k] = the k largest scores[b, :S] in descending order, ties to the lower
 *   index; vals (optional) their scores.  k <= S, k <= 1024.  Replaces the top-k of
 *   TopKSelector.select_from_input (xenc/topk_read.py:237-240).
 * xenc_gather_pages: out[g, j] = the slot row of flat index idx[g, j] (chunk idx / n_flat, slot
 *   idx % n_flat; chunk c on page chunk_page[c]) for j < k, zero rows for k <= j < kpad;
 *   out fp16 [G, kpad, d].  Out-of-range indices give zero rows.  The gathered pages form a
 *   one-chunk library per set whose read (route weight 1) is the read over the selected slots
 *   (xenc/topk_read.py:383-414).
 */
int xenc_select_scores(const float* q, int B, int n_q, int n_kv, int hd, const float* keys, int S,
                       const unsigned char* valid, int pool_mean, float* scores, long long ld_s,
                       void* stream);
int xenc_topk_rows(const float* scores, long long ld_s, int B, int S, int k, int* idx, float* vals,
                   long long ld_o, void* stream);
int xenc_gather_pages(const void* pages, int slots_per_page, long long page_stride, int d,
                      const int* chunk_page, int n_chunks, int n_flat, const int* idx,
                      long long ld_idx, int G, int k, int kpad, void* out, void* stream);

/*
 * ---- Op B serving step (per-request decode state on the device)
 * slots int32 [n_slots][4] = {op_start block, op_tokens, own_len, unused} per request slot; slot s
 * owns own-pool blocks [s * own_blocks, (s + 1) * own_blocks).  row_slot int32 [N]: the slot
 * decoded by row i (< 0: a padded row); a slot appears in at most one row per call.
 * xenc_decode_step, for each row i with slot s: p0 = slots[s].own_len;
 *   write_pos[i] = s * own_blocks * block_size + p0 (int64; -1 when p0 reached the capacity or for
 *   a padded row), own_len[i] = p0 + 1 (capped), slots[s].own_len = p0 + 1,
 *   op_len[i] = slots[s].op_tokens, op_bt[i][j] = op_start + j for j < ceil(op_tokens /
 *   block_size) else dummy_block (j < max_op_blocks), own_bt[i][j] = s * own_blocks + j.
 *   Padded rows get op_len = own_len = 0, dummy op blocks and own block 0.
 * xenc_own_rows_write: own pool rows write_pos[i] (block write_pos / block_size, slot
 *   write_pos % block_size) of own_k / own_v ([num_blocks, block_size, hkv, d], element strides
 *   sb, ss, sh, d contiguous) <- k_new / v_new [N, hkv, d] (strides s_n, s_h); 2-byte elements
 *   (fp16 or bf16), d % 8 == 0, 16-byte aligned; rows with write_pos < 0 are skipped.
 * Both allocate nothing and read nothing back, so a decode step (xenc_decode_step,
 * xenc_own_rows_write, xenc_paged_decode_joint) captures into one graph and replays step after
 * step.  Replaces the per-step host fill and copies of Static.fill / stage_step and the own-row
 * index_copy_ of read_static (xenc/d23_vllm_plugin.py:241-264, 433-457, 486-487).
 */
int xenc_decode_step(int N, const int* row_slot, int* slots, int n_slots, int own_blocks,
                     int block_size, int max_op_blocks, int dummy_block, int* op_bt,
                     long long ld_op_bt, int* op_len, int* own_bt, long long ld_own_bt,
                     int* own_len, long long* write_pos, void* stream);
int xenc_own_rows_write(int N, int hkv, int d, const void* k_new, const void* v_new, long long s_n,
                        long long s_h, void* own_k, void* own_v, long long sb, long long ss,
                        long long sh, int block_size, const long long* write_pos, void* stream);

/*
 * ---- D18 multi-document read: the attention core of lib_read (xenc/d18_library.py:63-90)
 * For reader row t, kv head h and query head g of its G = hq / hkv (GQA):
 *   document d (keys / values rows doc_ptr[d] .. doc_ptr[d+1]-1 of k_docs / v_docs [hkv][Ntot][hd],
 *   element strides s_dh, s_dn; dtype 0 fp16, 1 bf16, 2 fp32):
 *     s_d = scale * qd[d, t, hg] . K_d,   o_d = softmax([s_d ; s_own]) . [V_d ; V_own],
 *     r_d = logsumexp(s_d[skip:]), rmax_d = max(s_d[skip:])   (all of s_d when N_d <= skip)
 *   own rows (k_own / v_own fp32 [hkv][P + T][hd], strides s_oh, s_on): s_own = scale *
 *     qo[t, hg] . K_own[0 .. P + t] (causal);
 *   w = softmax_d(beta * r) over the top_k largest (top_k = 0 or >= D: all; ties to the lower
 *     index), or one-hot at force (>= 0), or wfix [D] (device, when force < 0 and wfix != NULL);
 *   out[t, hg, :] = sum_d w_d o_d.
 * qd [D][T][hq][hd] and qo [T][hq][hd] fp32 contiguous (the caller's RoPE rotations: document d
 * at N_d + P + t, own rows at P + t).  Outputs w, r, rmax [hkv][G][T][D] fp32, out [T][hq][hd]
 * fp32.  Each document's keys and the own rows are read in nsplit ranges (1..32) by separate
 * workgroups and merged in order.  Limits: 1 <= D <= 64, G <= 8, hd in {32, 64, 128, 256};
 * strides multiples of 16 bytes, row strides >= hd; doc_ptr int32 [D + 1] on the device.
 * workspace >= xenc_d18_workspace_bytes(T, hq, D, hd, nsplit) bytes of device memory, 16-byte
 * aligned (no zeroing needed).  Replaces the per-document loop of lib_read
 * (xenc/d18_library.py:63-90).
 */
size_t xenc_d18_workspace_bytes(int T, int hq, int n_docs, int hd, int nsplit);
int xenc_d18_read(int dtype, int T, int hq, int hkv, int hd, int n_docs, const float* qd,
                  const float* qo, const void* k_docs, const void* v_docs, long long s_dh,
                  long long s_dn, const int* doc_ptr, const float* k_own, const float* v_own,
                  long long s_oh, long long s_on, int P, float scale, int skip, float beta,
                  int top_k, int force, const float* wfix, int nsplit, float* out, float* w,
                  float* r, float* rmax, void* workspace, size_t workspace_bytes, void* stream);

/*
 * ---- Calibration (roofline denominators measured on the device; no counterpart in the reference)
 * xenc_calibrate_mfma: cus * waves_per_cu waves (waves_per_cu a multiple of 4) each run `rounds`
 *   rounds of 16 independent v_mfma_f32_32x32x16_f16 on operands read once from src (fp16, n_src
 *   16-byte vectors); out receives one float per lane (cus * waves_per_cu * 64 floats).
 *   FLOPs per launch: cus * waves_per_cu * rounds * 16 * 32768.
 * xenc_calibrate_stream: `blocks` workgroups of 256 threads read `bytes` of src once with 16-byte
 *   nontemporal loads (workgroup b a contiguous 1/blocks of it); out receives blocks * 256 floats.
 */
int xenc_calibrate_mfma(const void* src, int n_src, int waves_per_cu, int cus, int rounds, float* out,
                        void* stream);
int xenc_calibrate_stream(const void* src, long long bytes, int blocks, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* XENC_HIP_H */
