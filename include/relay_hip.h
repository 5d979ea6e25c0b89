/* relay_hip.h -- the C ABI of relay's MI355X (gfx950) backend.
 *
 * Two layers, both plain C: pointers, sizes and a hipStream_t passed as void*.
 *
 *  1. Kernel launchers (rh_*). Each takes device pointers that the caller owns and
 *     enqueues work on `stream` (NULL = the default stream). They return 0, or a
 *     nonzero code with rh_last_error() describing it (per thread). Shapes are checked
 *     on the host before anything is launched.
 *
 *  2. The backend object (relay_hip_backend_*): the whole forward pass of a Llama/Qwen2
 *     model over relay's paged KV cache, behind the same contract as relay's C++
 *     `Backend` interface (engine/include/relay/backend.h:43-81): forward() returns fp32
 *     logits, KV blocks can be read and written for the transfer engine, weights can be
 *     updated in place. The C++ class itself (relay::make_hip_backend) is declared in
 *     relay_amd/csrc/host/relay/backend.h for C++ callers such as relay's Engine.
 *
 * Conventions shared with relay (all cited files are in the reference tree):
 *  - KV cache layout per layer, for K and for V separately (kv_cache.h:20-37):
 *      [block][kv_head][slot][head_dim], fp16, element offset
 *      ((block * kv_heads + kv_head) * block_size + slot) * head_dim.
 *    Token position p of a sequence lives in block table[p / block_size], slot p % block_size.
 *  - Token metadata (cuda_kernels.cuh:16-21): for each of the T tokens of a step, pos[t]
 *    and seq[t] (its chunk); table_off[s] is where chunk s's block table starts in the
 *    concatenated `tables` array.
 *  - fp16 values are passed as void* holding IEEE binary16.
 */
#ifndef RELAY_HIP_H
#define RELAY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- errors ------------------------------------------------------------------ */

/* The message of the last failed call on this thread ("" if none). */
const char* rh_last_error(void);

/* 1 if a HIP device is present and usable, else 0 (never fails). */
int rh_device_available(void);

/* ---- attention over the paged cache ----------------------------------------------- */

/* Split-context decode attention ("flash-decoding") for single-token chunks, with the
 * log-sum-exp merge of the slices fused in (the last workgroup of a (token, kv head) to
 * finish merges its slices).
 * Replaces decode_attention_kernel<D,G> + decode_combine_kernel
 * (cuda_kernels.cuh:223-339, 341-362) and their launch (cuda_backend.cu:677-686).
 *
 *  q           fp16, row t at q + t * q_row_stride (elements), heads * head_dim values
 *  kpool/vpool fp16 paged cache of ONE layer
 *  dec_meta    int32 [n_dec][4], 16-byte aligned: per decode token (its row t in q and out,
 *              its context length = position + 1, the offset of its block table in
 *              `tables`, unused). The same facts relay's kernel reads through
 *              pos / seq / table_off (cuda_kernels.cuh:16-26), packed so that a workgroup
 *              reaches its block table after one load.
 *  out         fp16, row t at out + t * out_row_stride, heads * head_dim values
 *  slice_keys  keys per split (relay uses 512); a multiple of rh_decode_chunk_keys(head_dim);
 *              rh_decode_slice_keys() picks one for a step's shape
 *  max_parts   >= ceil(max context / slice_keys) over the decode tokens
 *  part_o      fp32 scratch, n_dec * heads * max_parts * head_dim
 *  part_ml     fp32 scratch, n_dec * heads * max_parts * 2
 *  counters    int32 scratch, n_dec * kv_heads * ceil((heads / kv_heads) / 16), all ZERO
 *              before the first call; every call leaves them zero again. Calls that share
 *              counters must not overlap in time (same stream is fine)
 *  scale       softmax scale (1/sqrt(head_dim) in relay)
 * head_dim in {16, 32, 64, 128} (16 computed at width 32); any group size (query heads are
 * processed 16 at a time). */
int rh_paged_decode_attention(const void* q, int64_t q_row_stride, const void* kpool, const void* vpool,
                              const int* dec_meta, const int* tables, int n_dec, int heads, int kv_heads,
                              int head_dim, int block_size, int slice_keys, int max_parts, float scale,
                              float* part_o, float* part_ml, int* counters, void* out, int64_t out_row_stride,
                              void* stream);

/* rh_paged_decode_attention without caller scratch, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in relay. The slice partials and arrival counters live in a
 * static device array of rh_decode_noalloc_scratch_bytes() (16 MiB), held on each GPU the
 * library runs on until the process ends; the call allocates nothing. Limits:
 * n_dec * kv_heads * ceil(group / 16) <= 16384 and
 * 4 * (16384 + n_dec * heads * max_parts * (head_dim + 2)) <= 16 MiB, else an error.
 * Every call on a GPU shares that GPU's array: calls that overlap in time on one GPU
 * (different streams, threads or processes' graphs) race and must not be made. */
int rh_paged_decode_attention_noalloc(const void* q, int64_t q_row_stride, const void* kpool, const void* vpool,
                                      const int* dec_meta, const int* tables, int n_dec, int heads, int kv_heads,
                                      int head_dim, int block_size, int slice_keys, int max_parts, float scale,
                                      void* out, int64_t out_row_stride, void* stream);
size_t rh_decode_noalloc_scratch_bytes(void);

/* Keys per streaming stage of a wave (16 KB of K+V at head_dim 64 and 128, 8 KB at 32): 128 at
 * head_dim 16 and 32, 64 at 64, 32 at 128; -1 otherwise. */
int rh_decode_chunk_keys(int head_dim);

/* The slice_keys rh_paged_decode_attention runs fastest with on MI355X for a step of n_dec
 * decode tokens whose longest context is max_ctx: whole contexts per workgroup unless
 * that leaves CUs idle. */
int rh_decode_slice_keys(int n_dec, int kv_heads, int group, int head_dim, int max_ctx);

/* Flash prefill attention for multi-token chunks: causal attention of each chunk's query
 * rows against keys 0..pos of their own sequence, all read from the paged cache (a chunk
 * at an offset sees the earlier chunks' keys).
 * Replaces flash_prefill_kernel<D> (cuda_kernels.cuh:37-178) and its launch
 * (cuda_backend.cu:528-545, 669-676, 689-693).
 *  work        int32[n_work][8] records from rh_prefill_plan (16-byte aligned): one or
 *              two blocks of rows (first row, rows, first position) and the chunk's
 *              block-table offset
 *  tables      the block tables the records' offsets point into
 *  scale       scores are scale * q.k; the kernel works in the exp2 domain and rounds
 *              q * scale * log2(e) to fp16 once more, unless that multiplier is exactly 1
 *              (scale = ln 2): then q is taken as already scaled, as the q writers'
 *              q_scale leaves it (the backend's path)
 * head_dim in {16, 32, 64, 128} (16 computed at width 32). */
int rh_flash_prefill(const void* q, int64_t q_row_stride, const void* kpool, const void* vpool, const int* tables,
                     const int* work, int n_work, int heads, int kv_heads, int head_dim, int block_size, float scale,
                     void* out, int64_t out_row_stride, void* stream);

/* Host-side: cut the step's prefill chunks (chunk s = rows chunk_t0[s] .. +chunk_rows[s]-1
 * of q/out at positions chunk_pos0[s].., block table at chunk_table_off[s]) into
 * rh_flash_prefill work records: blocks of up to rh_prefill_tile_rows() rows, paired
 * light-with-heavy when the step is large, heaviest first. Returns the record count, or a
 * negative error code if more than `capacity` records are needed (n_chunks + rows / 128 + 1
 * always suffice). Relay cuts the same row tiles in its launch (cuda_backend.cu:528-545),
 * one block each, in chunk order. */
int rh_prefill_plan(const int* chunk_t0, const int* chunk_rows, const int* chunk_pos0, const int* chunk_table_off,
                    int n_chunks, int heads, int* work, int capacity);

/* Query rows per prefill block. */
int rh_prefill_tile_rows(void);

/* Reference attention for any token (decode or prefill), any head_dim <= 256 and any
 * group size: one workgroup per (token, head), fp32 throughout. The role of relay's M0
 * kernel (cuda_backend.cu:200-243, RELAY_CUDA_ATTENTION=m0): what the fast kernels are
 * compared with on the GPU, and the path for head sizes they do not cover.
 *  q           fp32 (the RoPE'd rows of the qkv buffer), row t at q + t * q_row_stride
 *  tokens[n]   which tokens to compute (NULL: tokens 0..n-1) */
int rh_reference_attention(const float* q, int64_t q_row_stride, const void* kpool, const void* vpool,
                           const int* pos, const int* seq, const int* table_off, const int* tables,
                           const int* tokens, int n, int heads, int kv_heads, int head_dim, int block_size,
                           float scale, void* out, int64_t out_row_stride, void* stream);

/* ---- weight-only int8 ----------------------------------------------------------- */

/* y[t, n] = scale[n] * sum_k W8[n, k] * x[t, k]  (+ beta * y[t, n] when beta != 0), for
 * 1 <= T <= 64 tokens (relay's GEMV takes up to 8). W8 int8 [N, K] rows ldw bytes apart
 * (K <= ldw < 2^21, a multiple of 16; relay's layout is ldw = K); x fp16 [T, K]; y fp32 [T, N].
 * scale is fp32 [N] (scale_is_f16 = 0, relay's quantizer) or fp16 [N] (scale_is_f16 = 1).
 * K must be a multiple of 16 and W8 / x 16-byte aligned.
 * Replaces gemv_int8_kernel<8> (cuda_kernels.cuh:378-430) and its dispatch
 * (cuda_backend.cu:711-718). */
int rh_gemv_int8(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16, const void* x, float* y,
                 int T, int K, int N, float beta, void* stream);

/* The row stride (bytes) rh_gemv_int8 streams fastest for rows of K int8 values: K rounded
 * up to 16, plus 256 when that is a multiple of 2048 (rows a power-of-two multiple of 2 KB
 * apart put every load of a 16-row tile on the same HBM channels). No counterpart in
 * relay, whose int8 matrices are dense (cuda_backend.cu:282-304). */
int64_t rh_gemv_int8_row_stride(int K);

/* Largest T rh_gemv_int8 takes. */
int rh_gemv_int8_max_tokens(void);

/* rh_gemv_int8 with the producer of x or qkv_post folded in, for 1 <= T <= 16 (1 <= T <= 32
 * for rh_gemv_int8_qkv, which folds in only qkv_post) (no
 * counterpart in relay, where rms_norm_kernel, silu_mul_kernel and qkv_post run as their own
 * launches around the GEMV, cuda_backend.cu:575-591): the int8 counterparts of
 * rh_gemv_f16_rmsnorm, rh_gemv_f16_silu, rh_gemv_f16_qkv and rh_gemv_f16_rmsnorm_qkv, with
 * their operands and limits (rh_gemv_f16_fused_fits(T, K) for the fused producers) and
 * rh_gemv_int8's weights and scales. At 1-16 tokens the plain rh_gemv_int8 and the RMSNorm
 * and qkv forms run whole-line kernels whose row groups and wave splits can differ, and
 * rh_gemv_int8_silu runs the 16-row tile, so the fused results agree with the launches they
 * replace within the fp32 accumulation bound 4 * K * 2^-24 * sum|w * x|. */
int rh_gemv_int8_rmsnorm(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16, const float* x,
                         const float* norm_w, float eps, float* y, int T, int K, int N, float beta, void* stream);
int rh_gemv_int8_silu(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16, const float* gu, float* y,
                      int T, int K, int N, float beta, void* stream);
int rh_gemv_int8_qkv(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16, const void* x, float* qkv,
                     int T, int K, const float* bias, const float* inv_freq, const int* pos, const int* seq,
                     const int* table_off, const int* tables, void* kpool, void* vpool, void* q_out, float q_scale,
                     int heads, int kv_heads, int head_dim, int block_size, void* stream);
int rh_gemv_int8_rmsnorm_qkv(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16, const float* x,
                             const float* norm_w, float eps, float* qkv, int T, int K, const float* bias,
                             const float* inv_freq, const int* pos, const int* seq, const int* table_off,
                             const int* tables, void* kpool, void* vpool, void* q_out, float q_scale, int heads,
                             int kv_heads, int head_dim, int block_size, void* stream);

/* act[t, a] = fp16(silu(g) * u), g and u the rows a and I + a of rh_gemv_int8's product of
 * the fused gate/up matrix W8 [2 I, K] (scale [2 I]) with x fp16 [T, K], for 1 <= T <= 16;
 * act fp16 [T, I]. At 1-8 tokens the same bits as rh_gemv_int8 into an fp32 [T, 2 I] buffer
 * followed by rh_silu_mul, in one launch (each workgroup holds both halves of its
 * outputs); at 9-16 tokens the whole-line kernel, whose sums agree with rh_gemv_int8's within
 * the fp32 accumulation bound. No counterpart in relay (gemm then silu_mul_kernel,
 * cuda_backend.cu:590-591). */
int rh_gemv_int8_gate_up_silu(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16, const void* x,
                              void* act, int T, int K, int I, void* stream);

/* The fp16 counterpart, 1 <= T <= 32: act[t, a] = fp16(silu(g) * u) of the fused gate/up
 * matrix W16 [2 I, K] (rows ldw elements apart) with x fp16 [T, K], on the whole-line kernel
 * with SiLU·mul in its epilogue; agrees with rh_gemv_f16 + rh_silu_mul within the fp32
 * accumulation bound. No counterpart in relay (cublasGemmEx then silu_mul_kernel,
 * cuda_backend.cu:588-589). */
int rh_gemv_f16_gate_up_silu(const void* w16, int64_t ldw, const void* x, void* act, int T, int K, int I,
                             void* stream);

/* rh_gemv_int8_gate_up_silu with relay's RMSNorm of x folded in: act[t, a] = fp16(silu(g) *
 * u) of the product with xn = fp16(norm_w * (x * 1/sqrt(mean(x^2) + eps))), x fp32 [T, K] (the
 * residual stream), norm_w fp32 [K], 1 <= T <= 8, T * (K + 8) * 2 bytes <= 64 KiB. Where the
 * launch has >= 256 workgroups (I >= 2041) the bytes equal rh_rmsnorm followed by
 * rh_gemv_int8_gate_up_silu; below that the waves split K differently and the sums agree
 * within the fp32 accumulation bound. Every workgroup normalises x itself, so this pays
 * only while the (I + 7) / 8 workgroups fit one round on the CUs. No counterpart in relay
 * (rms_norm_kernel, gemm and silu_mul_kernel, cuda_backend.cu:587-589). */
int rh_gemv_int8_rmsnorm_gate_up_silu(const int8_t* w8, int64_t ldw, const void* scale, int scale_is_f16, const float* x,
                                      const float* norm_w, float eps, void* act, int T, int K, int I, void* stream);

/* y[t, n] = sum_k W16[n, k] * x[t, k]  (+ beta * y[t, n] when beta != 0), for 1 <= T <= 32:
 * the dense projection at decode batch sizes. W16 fp16 [N, K] rows ldw elements apart
 * (ldw >= K, a multiple of 8); x fp16 [T, K]; y fp32 [T, N]; K a multiple of 16; W16 and x
 * 16-byte aligned. fp32 accumulation of exact fp16 products in a fixed order.
 * Replaces cublasGemmEx (cuda_backend.cu:726-730) where T is small. */
int rh_gemv_f16(const void* w16, int64_t ldw, const void* x, float* y, int T, int K, int N, float beta,
                void* stream);

/* rh_gemv_f16 with K cut into ksplit ranges (1 <= ksplit <= 8, at most one per 64 values of
 * K), each its own workgroup, so that small-N products still cover the GPU. Partial sums go
 * to workspace (fp32, ksplit * T * N values) and the last workgroup of each 16-row tile to
 * finish adds them in range order (deterministic); counters holds ceil(N / 16) ints that
 * must be zero before the first call (each call leaves them zero). Calls that share a
 * workspace or counters must not overlap. ksplit = 1 is rh_gemv_f16 (workspace and
 * counters unused). No counterpart in relay (cublasGemmEx, cuda_backend.cu:726-730). */
int rh_gemv_f16_splitk(const void* w16, int64_t ldw, const void* x, float* y, int T, int K, int N, float beta,
                       int ksplit, float* workspace, int* counters, void* stream);

/* The ksplit rh_gemv_f16_splitk is fastest with for this shape (measured on MI355X). */
int rh_gemv_f16_split_plan(int T, int K, int N);

/* rh_gemv_f16 with the producer of x folded in (no counterpart in relay, where
 * rms_norm_kernel / silu_mul_kernel run as their own launches before the GEMM,
 * cuda_backend.cu:576-591). Each workgroup computes x for all T tokens into LDS:
 *   _rmsnorm: x fp32 [T, K] -> fp16(norm_w[k] * (x * 1/sqrt(mean_k(x^2) + eps))), the row's
 *             sum of squares in double (rh_rmsnorm's arithmetic);
 *   _silu:    gu fp32 [T, 2K] (gate | up) -> fp16(g / (1 + exp(-g)) * u) (rh_silu_mul's).
 * Requires rh_gemv_f16_fused_fits(T, K) (T * (K + 8) fp16 values fit 64 KB of LDS).
 * These (and rh_gemv_f16_qkv / _rmsnorm_qkv) run a whole-line kernel whose row groups and
 * wave split can differ from rh_gemv_f16's, so they agree with the two-launch chain within
 * the fp32 accumulation bound. */
int rh_gemv_f16_rmsnorm(const void* w16, int64_t ldw, const float* x, const float* norm_w, float eps, float* y,
                        int T, int K, int N, float beta, void* stream);
int rh_gemv_f16_silu(const void* w16, int64_t ldw, const float* gu, float* y, int T, int K, int N, float beta,
                     void* stream);
int rh_gemv_f16_fused_fits(int T, int K);

/* rh_gemv_f16_rmsnorm of the fused qkv projection (N = (heads + 2 kv_heads) head_dim) with
 * rh_qkv_post folded in as its epilogue: qkv fp32 [T, N] gets the same values, k and v rows
 * go into the paged cache and q to q_out (may be NULL) exactly as rh_qkv_post writes them
 * (relay runs rms_norm, the GEMM and qkv_post as three launches, cuda_backend.cu:575-578).
 * head_dim a multiple of 16; the limits of rh_gemv_f16_rmsnorm. */
int rh_gemv_f16_rmsnorm_qkv(const void* w16, int64_t ldw, const float* x, const float* norm_w, float eps,
                            float* qkv, int T, int K, const float* bias, const float* inv_freq, const int* pos,
                            const int* seq, const int* table_off, const int* tables, void* kpool, void* vpool,
                            void* q_out, float q_scale, int heads, int kv_heads, int head_dim, int block_size,
                            void* stream);

/* The same with x already fp16 [T, K] (no normalisation): rh_gemv_f16 then rh_qkv_post in
 * one launch, for the token counts where the RMSNorm cannot be folded in (1 <= T <= 32).
 * No counterpart in relay (cuda_backend.cu:577-578 are two launches). */
int rh_gemv_f16_qkv(const void* w16, int64_t ldw, const void* x, float* qkv, int T, int K, const float* bias,
                    const float* inv_freq, const int* pos, const int* seq, const int* table_off, const int* tables,
                    void* kpool, void* vpool, void* q_out, float q_scale, int heads, int kv_heads, int head_dim,
                    int block_size, void* stream);

/* Largest T rh_gemv_f16 takes. */
int rh_gemv_f16_max_tokens(void);

/* y[t, n] = scale[n] * sum_k W8[n, k] * x[t, k]  (+ beta * y[t, n] when beta != 0), any T >= 0:
 * the weight-only int8 product above the GEMV's token limit, on the matrix cores with the
 * int8 weights read once. W8 [N, K] rows ldw bytes apart (ldw >= K, a multiple of 16),
 * scale fp32 [N], x fp16 [T, K], y fp32 [T, N]; K a multiple of 64; W8 and x 16-byte
 * aligned. Same function as rh_gemv_int8 (fp32 sums of exact products, then the scale).
 * Replaces relay's dequantize + cublasGemmEx for T above the GEMV limit
 * (cuda_backend.cu:718-722). */
int rh_gemm_w8(const int8_t* w8, int64_t ldw, const float* scale, const void* x, float* y, int T, int K, int N,
               float beta, void* stream);

/* rh_gemm_w8 with K cut into ksplit ranges (1 <= ksplit <= 8, at most K / 64) so that
 * narrow matrices fill the GPU: each range writes its raw sums to workspace (fp32,
 * ksplit * T * N values, N a multiple of 4) and a second launch adds them in range order
 * before the scale and beta (deterministic, independent of timing). Calls sharing a
 * workspace must not overlap. rh_gemm_w8_plan(T, K, N) gives the split of the plan for the
 * shape (-1 if K is not a positive multiple of 64): above 64 tokens with K a multiple of
 * 128, the minimum of a timing model fitted to measurements over the kernels (128 x 128 and
 * 128 x 96 tiles on 128-k steps, 256 x 96 on 64-k steps) and 1-8 ranges; otherwise the
 * 128 x 128 or 256 x 96 tile on 64-k steps. rh_gemm_w8_kernel(T, K, N, ksplit) names the
 * kernel rh_gemm_w8_split runs for that split (0: 128 x 128 on 64-k steps, 1: 256 x 96,
 * 2: 128 x 128 on 128-k steps, 3: 128 x 96 on 128-k steps; -1 for bad arguments); the
 * kernels differ in the order in which each MFMA adds up its 16 k. No counterpart in
 * relay, which dequantizes the whole matrix and calls cublasGemmEx
 * (cuda_backend.cu:718-722). */
int rh_gemm_w8_split(const int8_t* w8, int64_t ldw, const float* scale, const void* x, float* y, int T, int K,
                     int N, float beta, int ksplit, float* workspace, void* stream);
int rh_gemm_w8_plan(int T, int K, int N);
int rh_gemm_w8_kernel(int T, int K, int N, int ksplit);

/* act[t, a] = fp16(silu(g) * u), g and u the rows a and I + a of rh_gemm_w8's product of
 * the fused gate/up matrix W8 [2 I, K] (scale fp32 [2 I]) with x fp16 [T, K]; act fp16
 * [T, I]. Runs the 256 x 96 tile (kernel 1 of rh_gemm_w8_kernel) unsplit with each
 * workgroup holding the gate and up rows of 128 outputs, so where rh_gemm_w8_kernel(T, K,
 * 2 I, 1) is 1 the bytes equal rh_gemm_w8 into an fp32 [T, 2 I] buffer followed by
 * rh_silu_mul, in one launch and without the fp32 buffer. Requires (I + 256) * ldw < 2^31.
 * No counterpart in relay (dequantize + cublasGemmEx, then silu_mul_kernel,
 * cuda_backend.cu:588-589, 718-722). */
int rh_gemm_w8_gate_up_silu(const int8_t* w8, int64_t ldw, const float* scale, const void* x, void* act, int T, int K,
                            int I, void* stream);

/* rh_gemm_w8 for 1 <= T <= 64 with a 128-row x 32-token tile (64 tokens above 32) and K cut
 * into ksplit ranges (1 <= ksplit <= 8, at most K / 64), so that decode batches of 17-64
 * tokens read the int8 weights once on enough workgroups: 128-k steps where K is a multiple
 * of 128 and ksplit <= K / 128, 64-k steps otherwise; workspace as for
 * rh_gemm_w8_split. No counterpart in relay (dequantize + cublasGemmEx,
 * cuda_backend.cu:718-722). */
int rh_gemm_w8_skinny(const int8_t* w8, int64_t ldw, const float* scale, const void* x, float* y, int T, int K, int N,
                      float beta, int ksplit, float* workspace, void* stream);

/* The first half of a split int8 product, for consumers that merge it themselves: the raw
 * sums of ksplit K ranges (2 <= ksplit <= 8, at most K / 64) into workspace [ksplit][T][N]
 * (N a multiple of 4), with the kernel rh_gemm_w8_skinny (T <= 64) or rh_gemm_w8_split
 * (rh_gemm_w8_kernel) runs for this T and split; no scale is applied. The merges below then add the ranges in order and apply
 * the scale, with the arithmetic of the two-launch chain (same bits). */
int rh_gemm_w8_partials(const int8_t* w8, int64_t ldw, const void* x, int T, int K, int N, int ksplit,
                        float* workspace, void* stream);
/* The split for rh_gemm_w8_partials when the consumer merges (-1 for bad arguments): the
 * rh_gemm_w8_plan split, except above 64 tokens where that plan runs the product unsplit on
 * fewer than 256 workgroups; there the K ranges the timing model prices lowest with the
 * merge done by the consumer (its extra partial reads only). No counterpart in relay. */
int rh_gemm_w8_partials_plan(int T, int K, int N);

/* act[t, i] = silu(g) * up of the merged gate_up partials (rows [0, I) gate, [I, 2I) up;
 * act fp16 [T, I], I a multiple of 8): rh_gemm_w8_skinny's merge followed by rh_silu_mul in
 * one launch (relay: silu_mul_kernel after the GEMM, cuda_backend.cu:588-589). */
int rh_w8_merge_silu(const float* workspace, int ksplit, int T, int I, const float* scale, void* act, void* stream);

/* x[t] += merged partials (beta = 1), then out = RMSNorm(x[t]) * norm_w (fp16 [T, H]): a
 * residual projection's merge, the residual add and the following RMSNorm in one launch,
 * with rh_rmsnorm's arithmetic (relay: rmsnorm_kernel after the GEMM, cuda_backend.cu:575,
 * 586-587). Also serves the o projection and the MLP's RMSNorm. H must satisfy rh_w8_merge_rmsnorm_fits (a multiple of 4, at
 * most 4096). */
int rh_w8_merge_rmsnorm(const float* workspace, int ksplit, int T, int H, const float* scale, float* x,
                        const float* norm_w, float eps, void* out, void* stream);
int rh_w8_merge_rmsnorm_fits(int H);

/* The ksplit rh_gemm_w8_skinny uses for this shape (-1 outside its limits). */
int rh_gemm_w8_split_plan(int T, int K, int N);

/* Per-row symmetric int8 quantization of an fp32 matrix [N, K] on the device:
 * scale[n] = max_k |w[n, k]| / 127 (1 if the row is all zero), q = round-half-even(w / scale),
 * q rows ldq bytes apart (ldq >= K; the bytes past K are not written).
 * Same values as the reference's host quantizer (cuda_backend.cu:282-304). */
int rh_quantize_int8(const float* w, int N, int K, int8_t* q, int64_t ldq, float* scale, void* stream);

/* W16[n, k] = fp16(W8[n, k] * scale[n]) for a whole [N, K] matrix (W8 rows ldw bytes apart,
 * W16 dense), the T > 16 path. Replaces dequant_int8_kernel (cuda_kernels.cuh:432-436). */
int rh_dequant_int8(const int8_t* w8, int64_t ldw, const float* scale, int N, int K, void* w16, void* stream);

/* ---- the rest of a transformer layer ------------------------------------------------ */

/* fp32 -> fp16, round to nearest even (bit-identical to relay's f32_to_f16,
 * safetensors.cpp:65-89). Replaces f32_to_f16_kernel (cuda_backend.cu:112-116). */
int rh_f32_to_f16(const float* in, void* out, size_t n, void* stream);

/* x[t, :] = fp32(table[tokens[t], :]), table fp16 [vocab, H]. (cuda_backend.cu:150-154) */
int rh_embed(const int* tokens, int T, const void* table, int H, float* x, void* stream);

/* out[r, :] = fp16(w * (x[rows[r], :] * rsqrt(mean(x^2) + eps))), rows NULL = r itself.
 * (cuda_backend.cu:157-167) */
int rh_rmsnorm(const float* x, const int* rows, int R, const float* w, int H, float eps, void* out, void* stream);

/* Per token: qkv row += bias (if not NULL); RoPE on the q and k heads (pairs (i, i + D/2),
 * angle pos * inv_freq[i]); k and v written as fp16 into the paged cache; q written as
 * fp16(q * q_scale) to q_out (row stride heads * head_dim; may be NULL). q_scale = 1 is the
 * plain copy; the backend passes softmax scale * log2(e), so that the attention kernels get
 * queries already in their exp2 domain with one rounding (and are called with scale = ln 2).
 * Every q_out writer below takes q_scale the same way. (cuda_backend.cu:171-198) */
int rh_qkv_post(float* qkv, int T, const float* bias, const float* inv_freq, const int* pos, const int* seq,
                const int* table_off, const int* tables, void* kpool, void* vpool, void* q_out, float q_scale,
                int heads, int kv_heads, int head_dim, int block_size, void* stream);

/* rh_qkv_post without the fp32 write-back: the same q (fp16, to q_out, required) and cache
 * rows, qkv left as it is. For callers that read only q_out and the cache afterwards (the
 * fast attention kernels); saves the fp32 rewrite of every q/k/v value (21 MB per layer for
 * a 2048-token TinyLlama prefill). No counterpart in relay (qkv_post_kernel rewrites qkv in
 * place, cuda_backend.cu:171-198). */
int rh_qkv_post_to_cache(const float* qkv, int T, const float* bias, const float* inv_freq, const int* pos,
                         const int* seq, const int* table_off, const int* tables, void* kpool, void* vpool,
                         void* q_out, float q_scale, int heads, int kv_heads, int head_dim, int block_size,
                         void* stream);

/* act[t, i] = fp16(g * sigmoid(g) * u), g = gu[t, i], u = gu[t, I + i]. (cuda_backend.cu:245-253) */
int rh_silu_mul(const float* gu, int T, int I, void* act, void* stream);

/* Pack (gather) or unpack (scatter) one layer's blocks: buf = [K of each listed block]
 * [V of each listed block], block_bytes a multiple of 16. (cuda_backend.cu:257-270) */
int rh_kv_gather(const void* kpool, const void* vpool, const int* blocks, int n, size_t block_bytes, void* buf,
                 void* stream);
int rh_kv_scatter(void* kpool, void* vpool, const int* blocks, int n, size_t block_bytes, const void* buf,
                  void* stream);

/* Fills out[i] (i < n) with fp16 / fp32 draws of mean + std * N(0, 1) from the
 * counter-based generator of rh_synth_normal_f32 (seed, stream, counter i). */
int rh_fill_normal_f16(void* out, size_t n, uint64_t seed, uint64_t stream_id, float mean, float std, void* stream);
int rh_fill_normal_f32(float* out, size_t n, uint64_t seed, uint64_t stream_id, float mean, float std, void* stream);

/* ---- synthetic inputs (host) ------------------------------------------------------ */

/* out[i] = mean + std * z_i, z_i ~ N(0, 1) from splitmix64(seed, stream_id, i) and
 * Box-Muller in double precision. Deterministic; multithreaded. */
void rh_synth_normal_f32(float* out, size_t n, uint64_t seed, uint64_t stream_id, float mean, float std);

/* ---- the backend object ------------------------------------------------------------ */

/* Model hyperparameters (relay's ModelConfig, config.h). rope_scaling_llama3 = 1 selects
 * Llama 3 frequency scaling with the four rope_* fields (config.cpp:79-109). */
typedef struct rh_model_config {
  int hidden, intermediate, layers, heads, kv_heads, head_dim, vocab, tie_embeddings, qkv_bias;
  int rope_scaling_llama3;
  double rms_eps, rope_theta, rope_factor, rope_low_freq_factor, rope_high_freq_factor, rope_original_max_position;
} rh_model_config;

/* Host fp32 weights in relay's fused layout (weights.h:13-31); pointers per layer.
 * lm_head NULL when tied to embed; bqkv[l] NULL without q/k/v bias. */
typedef struct rh_host_weights {
  const float* embed;      /* [vocab, hidden] */
  const float* final_norm; /* [hidden] */
  const float* lm_head;    /* [vocab, hidden] or NULL */
  const float* const* attn_norm; /* [layers] of [hidden] */
  const float* const* wqkv;      /* [layers] of [q_dim + 2 kv_dim, hidden] */
  const float* const* bqkv;      /* [layers] of [q_dim + 2 kv_dim] or NULL */
  const float* const* wo;        /* [layers] of [hidden, q_dim] */
  const float* const* mlp_norm;  /* [layers] of [hidden] */
  const float* const* w_gate_up; /* [layers] of [2 intermediate, hidden] */
  const float* const* w_down;    /* [layers] of [hidden, intermediate] */
} rh_host_weights;

/* Options (relay's CudaOptions, backend.h:85-94). reference_attention: the reference
 * kernel everywhere (RELAY_HIP_ATTENTION=ref). int8_weights: weight-only int8 layers
 * (RELAY_HIP_INT8=1). */
typedef struct rh_backend_options {
  int reference_attention;
  int int8_weights;
} rh_backend_options;

/* The options from the environment. */
rh_backend_options rh_backend_options_from_env(void);

typedef struct relay_hip_backend relay_hip_backend;

/* make_hip_backend (the HIP twin of make_cuda_backend, backend.h:95-97). The weights are
 * copied to the device; the host arrays may be freed afterwards. NULL on failure. */
relay_hip_backend* relay_hip_backend_new(const rh_model_config* config, const rh_host_weights* weights,
                                         int num_blocks, int block_size, int device, int max_batch_tokens,
                                         int max_context, const rh_backend_options* options);

/* The same model with weights drawn on the device: every matrix and the embedding ~
 * N(0, std) in fp16 from rh_fill_normal_f16, norms 1, biases 0. For benchmarks of
 * models too large to build on the host. */
relay_hip_backend* relay_hip_backend_new_synthetic(const rh_model_config* config, uint64_t seed, float std,
                                                   int num_blocks, int block_size, int device,
                                                   int max_batch_tokens, int max_context,
                                                   const rh_backend_options* options);
void relay_hip_backend_free(relay_hip_backend* b);

/* Backend::forward (backend.h:50-52) over a batch given as flat arrays: chunk s has
 * n_tokens[s] tokens (taken in order from `tokens`), starts at start_pos[s], has the block
 * table of table_len[s] entries (taken in order from `tables`) and want_logits[s].
 * Logits rows go to `logits` (capacity logits_cap floats); returns the number of rows
 * (each vocab floats), or -1 on error. */
int relay_hip_backend_forward(relay_hip_backend* b, int n_seqs, const int* n_tokens, const int* tokens,
                              const int* start_pos, const int* table_len, const int* tables,
                              const int* want_logits, int all_logits, float* logits, size_t logits_cap);

/* KV block I/O (backend.h:54-72). Block bytes = kv_heads * block_size * head_dim * 2. */
size_t relay_hip_backend_kv_block_bytes(const relay_hip_backend* b);
int relay_hip_backend_read_kv_block(relay_hip_backend* b, int layer, int block, void* k_out, void* v_out);
int relay_hip_backend_write_kv_block(relay_hip_backend* b, int layer, int block, const void* k_in, const void* v_in);
int relay_hip_backend_read_kv_layer(relay_hip_backend* b, int layer, const int* blocks, int n, void* out);
int relay_hip_backend_write_kv_layer(relay_hip_backend* b, int layer, const int* blocks, int n, const void* in);
int relay_hip_backend_wait_kv_written(relay_hip_backend* b, int layer);

/* Backend::update_weight (backend.h:74-80): `name` as relay names weights, src fp32 in
 * host memory or device memory of any GPU. */
int relay_hip_backend_update_weight(relay_hip_backend* b, const char* name, const float* src, size_t n);

/* Fills every layer's K and V cache with N(0, std) fp16 draws (benchmarks that need a
 * filled cache without running the prompts). */
int relay_hip_backend_fill_kv_random(relay_hip_backend* b, uint64_t seed, float std);

/* Time in milliseconds of the last forward() measured on the device (HIP events around
 * the layer loop), for benchmarks. */
double relay_hip_backend_last_forward_ms(const relay_hip_backend* b);

#ifdef __cplusplus
}
#endif

#endif /* RELAY_HIP_H */
