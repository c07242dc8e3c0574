/*
 * fracture_hip.h — C ABI of libfracture_hip.so, an MI355X (gfx950) implementation of the
 * elementwise / reduction / TurboQuant hot path behind Fracture's `Backend` trait.
 *
 * Three groups of entry points:
 *
 *   1. Raw launchers `fhip_launch_*`: device pointers, int32 dims, asynchronous on the
 *      given stream, return 0 (hipSuccess) or a HIP error code. The first eight replace,
 *      one for one, the `launch_*` symbols that the reference's Rust code binds in
 *      backends/fracture-cuda/src/ffi.rs:141-274. They allocate nothing, except the two
 *      paged-attention launchers with the reference's signature, which has no workspace
 *      argument: those take their split partials from a stream-ordered allocation
 *      (hipMallocAsync / hipFreeAsync on the given stream); their `_ws` forms take a
 *      caller-owned workspace instead.
 *   2. A handle runtime `fhip_*` that mirrors the `Backend` trait
 *      (crates/fracture-core/src/backend.rs:8-223) over opaque tensor ids, plus the
 *      inherent `CudaBackend` API (backends/fracture-cuda/src/lib.rs:76-161). Calls return
 *      an FHIP_* status; `fhip_last_error()` gives the message of the calling thread's last
 *      failure, worded like the reference's `FractureError` strings.
 *   3. Host-only helpers (no GPU) for the TurboQuant tables the reference builds on the CPU
 *      (crates/fracture-core/src/turboquant.rs:99-438) and the RoPE frequency table
 *      (backends/fracture-cuda/src/lib.rs:133-155).
 *
 * Entry points marked "additive" have no counterpart in the reference's FFI; they cover the
 * ops the reference runs on the CPU (softmax/argmax in crates/fracture-generate/src/
 * sampling.rs:45-99), as two launches (add then rmsnorm, crates/fracture-engine/src/
 * engine.rs:692-697) or only from tests (dequantize).
 */
#ifndef FRACTURE_HIP_H
#define FRACTURE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A hipStream_t; NULL means the default (null) stream. */
typedef void* fhip_stream_t;

/* Status codes of the handle runtime; the names follow fracture_core::FractureError
 * (crates/fracture-core/src/error.rs:6-51). */
enum {
    FHIP_OK = 0,
    FHIP_ERR_BACKEND = 1,           /* FractureError::Backend          */
    FHIP_ERR_INVALID_SHAPE = 2,     /* FractureError::InvalidShape     */
    FHIP_ERR_TENSOR_NOT_FOUND = 3,  /* FractureError::TensorNotFound   */
    FHIP_ERR_OUT_OF_MEMORY = 4,     /* FractureError::OutOfMemory      */
    FHIP_ERR_UNSUPPORTED_DTYPE = 5, /* FractureError::UnsupportedDType */
    FHIP_ERR_GENERATION = 6         /* FractureError::Generation       */
};

/* Element types, in the order of fracture_core::DType (crates/fracture-core/src/dtype.rs:5-11). */
enum { FHIP_FP16 = 0, FHIP_FP32 = 1, FHIP_BF16 = 2, FHIP_INT8 = 3, FHIP_INT4 = 4 };

/* Flags written by the row argmax kernels (the sampler's NaN / Inf rejection,
 * crates/fracture-generate/src/sampling.rs:51-56). */
enum { FHIP_ROW_HAS_NAN = 1u, FHIP_ROW_HAS_INF = 2u };

/* Tokens per KV page (block) of the paged caches
 * (crates/fracture-engine/src/paged_kv_cache.rs:7, attention_paged_tq.cu:35). */
#define FHIP_PAGE_TOKENS 16

/* =====================================================================================
 * 1. Raw launchers
 * ===================================================================================== */

/* ffi.rs:142-150 `launch_rmsnorm`: out[r,:] = fp16(x * rsqrt(mean(x^2) + eps) * w), fp16. */
int fhip_launch_rmsnorm(void* output, const void* input, const void* weight, float eps, int rows,
                        int cols, fhip_stream_t stream);

/* ffi.rs:152-162 `launch_rope`: split-half rotary embedding in place on q [T,qh,hd] and
 * k [T,kvh,hd] (fp16); positions u32[T] and freq_table f32[hd/2] in device memory. */
int fhip_launch_rope(void* q, void* k, const uint32_t* positions, const float* freq_table,
                     int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                     fhip_stream_t stream);

/* ffi.rs:164-170 `launch_silu_mul`: out = fp16(silu(gate) * up), n elements. */
int fhip_launch_silu_mul(void* output, const void* gate, const void* up, int n,
                         fhip_stream_t stream);

/* ffi.rs:202-210 `launch_embedding`: out[t,:] = table[ids[t],:]; ids >= vocab give zeros. */
int fhip_launch_embedding(void* output, const void* table, const uint32_t* token_ids,
                          int num_tokens, int hidden_dim, int vocab_size, fhip_stream_t stream);

/* ffi.rs:212-218 `launch_add`: out = a + b, fp16 (round to nearest even). */
int fhip_launch_add(void* output, const void* a, const void* b, int n, fhip_stream_t stream);

/* ffi.rs:222-235 `launch_turboquant_compress`: per vector of input [N, kvh, hd] fp16:
 * norm -> normalize -> y = rotation @ x_hat -> nearest centroid (first minimum) -> MSB-first
 * bit-pack into packed_out [N, kvh*packed_dim_per_head]; norms_out [N, kvh] fp16.
 * bits in 1..8 (the reference accepts 2, 4, 8; 3 is the MSB-first bitstream generalization). */
int fhip_launch_turboquant_compress(const void* input, const float* rotation,
                                    const float* centroids, void* packed_out, void* norms_out,
                                    int num_tokens, int num_kv_heads, int head_dim, int n_levels,
                                    int bits, int packed_dim_per_head, fhip_stream_t stream);

/* ffi.rs:237-249 `launch_turboquant_decompress`: unpack -> centroid -> rotation^T @ y_hat ->
 * fp16(x_hat * norm). */
int fhip_launch_turboquant_decompress(const void* packed_in, const void* norms_in,
                                      const float* rotation, const float* centroids,
                                      void* output, int num_tokens, int num_kv_heads,
                                      int head_dim, int bits, int packed_dim_per_head,
                                      fhip_stream_t stream);

/* ffi.rs:251-274 `launch_attention_paged_tq`: causal GQA attention of q [T, qh, hd] fp16 over
 * TurboQuant pages given as per-block pointer arrays (device memory), with the query
 * pre-rotated by k_rotation and the output unrotated by v_rotation^T. Unlike the reference
 * kernel it keeps no kv_len-sized score row: kv_len may be up to 1,048,576 positions.
 * head_dim is a multiple of 8 up to 256; T up to 65535. The split partials come from a
 * stream-ordered allocation on `stream` (see fhip_launch_attention_paged_tq_ws). */
int fhip_launch_attention_paged_tq(void* output, const void* q, const int* block_table,
                                   const void** k_packed_ptrs, const void** k_norms_ptrs,
                                   const void** v_packed_ptrs, const void** v_norms_ptrs,
                                   const float* k_rotation, const float* v_rotation,
                                   const float* k_centroids, const float* v_centroids,
                                   int num_tokens, int num_q_heads, int num_kv_heads,
                                   int head_dim, int kv_len, int start_pos, int key_bits,
                                   int value_bits, int k_packed_dim_per_head,
                                   int v_packed_dim_per_head, fhip_stream_t stream);

/* ffi.rs:186-200 `launch_paged_attention` (attention_paged.cu:172-185): causal GQA attention
 * of q [T, qh, hd] fp16 over FP16 pages given as per-block pointer arrays (device memory,
 * indexed by the physical block ids of block_table), each block [16, kvh, hd] fp16. head_dim
 * is 1 to 256 (32, 64, 128 and 256 run MFMA kernels, other widths a generic one). Unlike the
 * reference kernel it keeps no kv_len-sized score row: a block table may describe up to
 * 1,048,576 positions. The split partials come from a stream-ordered allocation on `stream`
 * (see fhip_launch_paged_attention_ws). */
int fhip_launch_paged_attention(void* output, const void* q, const int* block_table,
                                const void** k_block_ptrs, const void** v_block_ptrs,
                                int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                                int kv_len, int start_pos, int num_blocks_in_seq,
                                fhip_stream_t stream);

/* ffi.rs:172-184 `launch_attention` (contiguous KV cache): not supported; returns
 * hipErrorNotSupported and launches nothing. The engine's caches are paged (engine.rs:671-680
 * dispatches through the cache manager to the paged launchers above); the symbol lets a
 * binding of the whole ffi.rs block link. */
int fhip_launch_attention(void* output, const void* q, const void* k_cache, const void* v_cache,
                          int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                          int kv_len, int start_pos, fhip_stream_t stream);

/* The GEMM of CudaBackend::matmul (cuda/src/backend.rs:75-128), which calls cuBLAS directly:
 * C[M, N] = A[M, K] · B[N, K]^T, row-major fp16 operands, fp32 accumulation, on the stream. */
int fhip_launch_matmul(void* c, const void* a, const void* b, int m, int n, int k,
                       fhip_stream_t stream);

/* --- additive raw launchers ---------------------------------------------------------- */

/* The two reference-signature paged-attention launchers above with a caller-owned workspace
 * for the split partials, so that no call allocates: workspace_bytes must be at least
 * fhip_attention_tq_workspace_bytes(num_tokens, num_q_heads, head_dim, ceil(kv_len / 16))
 * (TurboQuant; 1 block when kv_len is 0) or fhip_attention_paged_workspace_bytes(num_tokens,
 * num_q_heads, head_dim, max(num_blocks_in_seq, 1)) (FP16). Calls sharing a workspace must be
 * ordered on one stream. */
int fhip_launch_attention_paged_tq_ws(void* output, const void* q, const int* block_table,
                                      const void** k_packed_ptrs, const void** k_norms_ptrs,
                                      const void** v_packed_ptrs, const void** v_norms_ptrs,
                                      const float* k_rotation, const float* v_rotation,
                                      const float* k_centroids, const float* v_centroids,
                                      int num_tokens, int num_q_heads, int num_kv_heads,
                                      int head_dim, int kv_len, int start_pos, int key_bits,
                                      int value_bits, int k_packed_dim_per_head,
                                      int v_packed_dim_per_head, void* workspace,
                                      size_t workspace_bytes, fhip_stream_t stream);
int fhip_launch_paged_attention_ws(void* output, const void* q, const int* block_table,
                                   const void** k_block_ptrs, const void** v_block_ptrs,
                                   int num_tokens, int num_q_heads, int num_kv_heads,
                                   int head_dim, int kv_len, int start_pos,
                                   int num_blocks_in_seq, void* workspace,
                                   size_t workspace_bytes, fhip_stream_t stream);

/* fhip_launch_attention_paged_tq that allocates nothing and takes no workspace. It has no
 * counterpart in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The split
 * partials live in a static device array of FHIP_TQ_ATTN_SCRATCH_BYTES per GPU, loaded with
 * the library and held until the process ends; a call whose partials need more
 * (fhip_attention_tq_workspace_bytes(num_tokens, num_q_heads, head_dim, ceil(kv_len / 16)),
 * e.g. one decode token of 32 heads at head_dim 128 up to 1,048,576 positions) returns
 * hipErrorOutOfMemory and launches nothing. Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (different streams, or host threads enqueueing at once) race
 * on it and must be ordered by the caller. The kernels write every partial they read, so
 * nothing in the array needs to start at zero. The stream's device is used; the first call on
 * each device looks up the array's address there. */
#define FHIP_TQ_ATTN_SCRATCH_BYTES ((size_t)32 << 20)
int fhip_launch_attention_paged_tq_noalloc(void* output, const void* q, const int* block_table,
                                           const void** k_packed_ptrs, const void** k_norms_ptrs,
                                           const void** v_packed_ptrs, const void** v_norms_ptrs,
                                           const float* k_rotation, const float* v_rotation,
                                           const float* k_centroids, const float* v_centroids,
                                           int num_tokens, int num_q_heads, int num_kv_heads,
                                           int head_dim, int kv_len, int start_pos, int key_bits,
                                           int value_bits, int k_packed_dim_per_head,
                                           int v_packed_dim_per_head, fhip_stream_t stream);

/* dtype-generic forms of rmsnorm / add / silu_mul (FHIP_FP16, FHIP_BF16, FHIP_FP32). */
int fhip_launch_rmsnorm_ex(void* output, const void* input, const void* weight, float eps,
                           int rows, int cols, int dtype, fhip_stream_t stream);
int fhip_launch_add_ex(void* output, const void* a, const void* b, int64_t n, int dtype,
                       fhip_stream_t stream);
int fhip_launch_silu_mul_ex(void* output, const void* gate, const void* up, int64_t n,
                            int dtype, fhip_stream_t stream);
/* rope for FHIP_FP16 / FHIP_BF16 / FHIP_FP32 q and k. */
int fhip_launch_rope_ex(void* q, void* k, const uint32_t* positions, const float* freq_table,
                        int num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                        int dtype, fhip_stream_t stream);
/* embedding of rows of elem_bytes-sized elements (2 for fp16/bf16, 4 for fp32). */
int fhip_launch_embedding_ex(void* output, const void* table, const uint32_t* token_ids,
                             int num_tokens, int hidden_dim, int vocab_size, int elem_bytes,
                             fhip_stream_t stream);

/* Fused residual add + RMSNorm, one HBM pass: residual = dtype(residual + delta) (in place,
 * rounded before the norm reads it, as add.cu:13 then rmsnorm.cu:27 do), then
 * normed_out = dtype(residual * rsqrt(mean(residual^2) + eps) * weight). */
int fhip_launch_add_rmsnorm(void* residual, const void* delta, const void* weight, float eps,
                            void* normed_out, int rows, int cols, int dtype,
                            fhip_stream_t stream);

/* Row softmax / argmax over fp32 logits [rows, cols] (the sampler's greedy and softmax paths,
 * sampling.rs:45-82). argmax ties resolve to the LAST index (Iterator::max_by); flags_out
 * gets FHIP_ROW_HAS_NAN / FHIP_ROW_HAS_INF per row. probs = exp(l/T - max) / sum.
 * The workspace holds per-chunk partials; size it with fhip_rows_workspace_bytes. Calls
 * sharing a workspace must be ordered on one stream. Each op is two launches. */
size_t fhip_rows_workspace_bytes(int rows, int cols);
int fhip_launch_softmax_rows(const float* logits, float* probs, int rows, int cols,
                             float temperature, void* workspace, fhip_stream_t stream);
int fhip_launch_argmax_rows(const float* logits, int32_t* index_out, uint32_t* flags_out,
                            int rows, int cols, void* workspace, fhip_stream_t stream);
int fhip_launch_softmax_argmax_rows(const float* logits, float* probs, int32_t* index_out,
                                    uint32_t* flags_out, int rows, int cols, float temperature,
                                    void* workspace, fhip_stream_t stream);

/* TurboQuant quantize + pack of given fp32 rotated vectors y [rows, head_dim]: the code of
 * each coordinate is the first index minimising |y - c| in fp32 (turboquant_compress.cu:
 * 120-130), packed MSB-first. Bit-exact with the reference for any y and any centroids. */
int fhip_launch_tq_quantize_pack(const float* y, const float* centroids, int n_levels, int bits,
                                 void* packed_out, int rows, int head_dim,
                                 int packed_dim_per_head, fhip_stream_t stream);

/* The fp32 rotated unit vectors y and fp16 norms that fhip_launch_turboquant_compress
 * quantizes, for the same input (identical arithmetic). */
int fhip_launch_tq_rotate(const void* input, const float* rotation, float* y_out,
                          void* norms_out, int rows, int head_dim, fhip_stream_t stream);

/* Compress [N, kvh, hd] fp16 straight into 16-token pages of a contiguous pool:
 * token t goes to page page_ids[(first_pos + t) / 16], slot (first_pos + t) % 16, in the
 * layout of quantized_paged_kv_cache.rs:86-128 (packed [16, kvh*pd] u8, norms [16, kvh]
 * fp16) with pool strides page_packed_bytes / page_norm_bytes (bytes between pages). */
int fhip_launch_tq_compress_pages(const void* input, const float* rotation,
                                  const float* centroids, int n_levels, int bits,
                                  void* packed_pool, void* norms_pool, int64_t page_packed_bytes,
                                  int64_t page_norm_bytes, const int32_t* page_ids, int num_pages,
                                  int first_pos, int num_tokens, int num_kv_heads, int head_dim,
                                  fhip_stream_t stream);

/* The page writer for pages that are separate allocations, as QuantizedKvCacheManager
 * allocates them (quantized_paged_kv_cache.rs:82-133): packed_pages[p] / norm_pages[p]
 * (device arrays of num_pages addresses) hold page p's packed rows [16, kvh*pd] and norms
 * [16, kvh] fp16. Token t goes to page page_ids[(first_pos + t) / 16], slot
 * (first_pos + t) % 16; rows whose page id is outside [0, num_pages) are not written. */
int fhip_launch_tq_compress_page_ptrs(const void* input, const float* rotation,
                                      const float* centroids, int n_levels, int bits,
                                      void* const* packed_pages, void* const* norm_pages,
                                      const int32_t* page_ids, int num_pages, int first_pos,
                                      int num_tokens, int num_kv_heads, int head_dim,
                                      fhip_stream_t stream);

/* launch_turboquant_decompress with an explicit codebook size (codes index only the first
 * n_levels centroids; the reference form assumes 2^bits). */
int fhip_launch_tq_dequant(const void* packed_in, const void* norms_in, const float* rotation,
                           const float* centroids, int n_levels, void* output, int num_tokens,
                           int num_kv_heads, int head_dim, int bits, int packed_dim_per_head,
                           fhip_stream_t stream);

/* TurboQuant plan: what compress and dequantize derive from one rotation and codebook (the
 * per-layer TurboQuantConfig that QuantizedKvCacheManager uploads once,
 * quantized_paged_kv_cache.rs:137-170), built once on the device in the layouts the kernels
 * use: the nearest-centroid quantizer tables and the fp16 hi/lo rotation fragments. The
 * planned launchers produce bytes identical to the unplanned ones for the same rotation and
 * centroids, without rebuilding those per call. head_dim must be 128. create allocates the
 * plan's device memory (about 210 KB) and enqueues its build on `stream`; the rotation and
 * centroids may change after that build has run. destroy waits for the device to idle. */
typedef struct fhip_tq_plan fhip_tq_plan;
int fhip_tq_plan_create(const float* rotation, const float* centroids, int n_levels, int bits,
                        int head_dim, fhip_stream_t stream, fhip_tq_plan** out);
void fhip_tq_plan_destroy(fhip_tq_plan* plan);
int fhip_launch_tq_compress_planned(const fhip_tq_plan* plan, const void* input,
                                    void* packed_out, void* norms_out, int num_tokens,
                                    int num_kv_heads, fhip_stream_t stream);
int fhip_launch_tq_compress_pages_planned(const fhip_tq_plan* plan, const void* input,
                                          void* packed_pool, void* norms_pool,
                                          int64_t page_packed_bytes, int64_t page_norm_bytes,
                                          const int32_t* page_ids, int num_pages, int first_pos,
                                          int num_tokens, int num_kv_heads,
                                          fhip_stream_t stream);
int fhip_launch_tq_compress_page_ptrs_planned(const fhip_tq_plan* plan, const void* input,
                                              void* const* packed_pages,
                                              void* const* norm_pages, const int32_t* page_ids,
                                              int num_pages, int first_pos, int num_tokens,
                                              int num_kv_heads, fhip_stream_t stream);
int fhip_launch_tq_dequant_planned(const fhip_tq_plan* plan, const void* packed_in,
                                   const void* norms_in, void* output, int num_tokens,
                                   int num_kv_heads, fhip_stream_t stream);

/* One layer's keys and values in one launch (append_kv's two turboquant_compress calls,
 * quantized_paged_kv_cache.rs:417-497, and the two decompresses of a layer): half the
 * workgroups take the keys, half the values, each with its own plan, so the two tensors'
 * load ramps and tails overlap. Bytes and outputs are those of the single-tensor planned
 * launchers. Width pairs without a K+V kernel (anything but equal widths of 2, 3, 4 or 8 bits,
 * or 4-bit keys with 2-bit values) run as two launches. */
int fhip_launch_tq_compress_kv_planned(const fhip_tq_plan* kplan, const fhip_tq_plan* vplan,
                                       const void* k_input, const void* v_input,
                                       void* k_packed_out, void* k_norms_out,
                                       void* v_packed_out, void* v_norms_out, int num_tokens,
                                       int num_kv_heads, fhip_stream_t stream);
int fhip_launch_tq_compress_kv_page_ptrs_planned(
    const fhip_tq_plan* kplan, const fhip_tq_plan* vplan, const void* k_input,
    const void* v_input, void* const* k_packed_pages, void* const* k_norm_pages,
    void* const* v_packed_pages, void* const* v_norm_pages, const int32_t* page_ids,
    int num_pages, int first_pos, int num_tokens, int num_kv_heads, fhip_stream_t stream);
int fhip_launch_tq_dequant_kv_planned(const fhip_tq_plan* kplan, const fhip_tq_plan* vplan,
                                      const void* k_packed_in, const void* k_norms_in,
                                      const void* v_packed_in, const void* v_norms_in,
                                      void* k_output, void* v_output, int num_tokens,
                                      int num_kv_heads, fhip_stream_t stream);

/* Batched decode attention over a TurboQuant page pool: one query token per sequence,
 * q [B, qh, hd] fp16, block_table [B, max_blocks] int32 (physical page ids), seq_lens [B]
 * int32; pages in contiguous pools (strides in bytes between pages, each at least one page:
 * 16 * kvh * packed_dim or 16 * kvh * 2 bytes); positions whose page id is outside
 * [0, num_pages) are masked out. max_blocks is at least 1 (a zero-width table, a batch of
 * empty sequences only, is refused with hipErrorInvalidValue) and max_blocks * 16 at most
 * 1,048,576. Output [B, qh, hd] fp16 (zeros for an empty sequence); centroid tables hold
 * 2^bits entries.
 * The workspace holds split-K partials; size it with fhip_attention_tq_workspace_bytes. */
size_t fhip_attention_tq_workspace_bytes(int batch, int num_q_heads, int head_dim,
                                         int max_blocks);
int fhip_launch_attention_tq_decode(void* output, const void* q, const int32_t* block_table,
                                    const int32_t* seq_lens, int batch, int max_blocks,
                                    int num_pages, const void* k_packed_pool, const void* k_norms_pool,
                                    const void* v_packed_pool, const void* v_norms_pool,
                                    int64_t page_k_packed_bytes, int64_t page_k_norm_bytes,
                                    int64_t page_v_packed_bytes, int64_t page_v_norm_bytes,
                                    const float* k_rotation, const float* v_rotation,
                                    const float* k_centroids, const float* v_centroids,
                                    int num_q_heads, int num_kv_heads, int head_dim,
                                    int key_bits, int value_bits, void* workspace,
                                    fhip_stream_t stream);

/* fhip_launch_attention_tq_decode over pages that are separate allocations: page p's four
 * parts are at k_packed_ptrs[p], k_norms_ptrs[p], v_packed_ptrs[p], v_norms_ptrs[p] (device
 * arrays of num_pages addresses). Same workspace as fhip_launch_attention_tq_decode. */
int fhip_launch_attention_tq_decode_ptrs(void* output, const void* q, const int32_t* block_table,
                                         const int32_t* seq_lens, int batch, int max_blocks,
                                         int num_pages, const void** k_packed_ptrs,
                                         const void** k_norms_ptrs, const void** v_packed_ptrs,
                                         const void** v_norms_ptrs, const float* k_rotation,
                                         const float* v_rotation, const float* k_centroids,
                                         const float* v_centroids, int num_q_heads,
                                         int num_kv_heads, int head_dim, int key_bits,
                                         int value_bits, void* workspace, fhip_stream_t stream);

/* Batched decode attention over an FP16 page pool (the FP16 form of the call above, for
 * batched decode): q [B, qh, hd] fp16, block_table [B, max_blocks] int32, seq_lens [B] int32;
 * page p of K at k_pool + p * page_k_bytes holds [16, kvh, hd] fp16, likewise V; positions
 * whose page id is outside [0, num_pages) are masked out; max_blocks is at least 1, as above.
 * Output [B, qh, hd] fp16.
 * The workspace holds split partials; size it with fhip_attention_paged_workspace_bytes. */
size_t fhip_attention_paged_workspace_bytes(int batch, int num_q_heads, int head_dim,
                                            int max_blocks);
int fhip_launch_attention_paged_decode(void* output, const void* q, const int32_t* block_table,
                                       const int32_t* seq_lens, int batch, int max_blocks,
                                       int num_pages, const void* k_pool, const void* v_pool,
                                       int64_t page_k_bytes, int64_t page_v_bytes,
                                       int num_q_heads, int num_kv_heads, int head_dim,
                                       void* workspace, fhip_stream_t stream);

/* =====================================================================================
 * 2. Handle runtime (mirror of the Backend trait)
 * ===================================================================================== */

typedef struct fhip_backend fhip_backend;

/* fracture_core::DeviceTensor (crates/fracture-core/src/tensor.rs:13-18) by value:
 * an id, a row-major shape and a dtype. The backend resolves the id; callers never see
 * device pointers. */
#define FHIP_MAX_DIMS 8
typedef struct {
    uint64_t id;
    int32_t dtype;
    int32_t ndim;
    uint64_t shape[FHIP_MAX_DIMS];
} fhip_tensor;

/* Message of the calling thread's most recent failing call (empty if none). */
const char* fhip_last_error(void);

/* CudaBackend::new (lib.rs:76-114) / Drop (lib.rs:164-182). */
int fhip_backend_create(int device_id, fhip_backend** out);
void fhip_backend_destroy(fhip_backend* b);

/* CudaBackend::get_ptr (lib.rs:117-125) and ::stream (lib.rs:127-129). */
int fhip_get_ptr(fhip_backend* b, uint64_t id, void** out);
fhip_stream_t fhip_stream(fhip_backend* b);

/* CudaBackend::precompute_rope_freqs (lib.rs:133-155). */
int fhip_precompute_rope_freqs(fhip_backend* b, size_t head_dim, double theta);

/* Backend::alloc / free / copy_to_device / copy_to_host (backend.rs:11-20). */
int fhip_alloc(fhip_backend* b, const uint64_t* shape, int ndim, int dtype, fhip_tensor* out);
int fhip_free(fhip_backend* b, const fhip_tensor* t);
int fhip_copy_to_device(fhip_backend* b, const fhip_tensor* dst, const void* src, size_t src_len);
int fhip_copy_to_host(fhip_backend* b, const fhip_tensor* src, void* dst, size_t dst_len);

/* Backend::rmsnorm / rope / silu_mul / embedding / add / copy_rows (backend.rs:30-121). */
int fhip_rmsnorm(fhip_backend* b, const fhip_tensor* input, const fhip_tensor* weight, double eps,
                 const fhip_tensor* out);
int fhip_rope(fhip_backend* b, const fhip_tensor* q, const fhip_tensor* k,
              const uint32_t* positions, size_t num_positions, double theta, size_t head_dim);
int fhip_silu_mul(fhip_backend* b, const fhip_tensor* gate, const fhip_tensor* up,
                  const fhip_tensor* out);
int fhip_embedding(fhip_backend* b, const uint32_t* token_ids, size_t num_tokens,
                   const fhip_tensor* table, const fhip_tensor* out);
int fhip_add(fhip_backend* b, const fhip_tensor* a, const fhip_tensor* bt, const fhip_tensor* out);
int fhip_copy_rows(fhip_backend* b, const fhip_tensor* src, const fhip_tensor* dst,
                   size_t src_offset, size_t dst_offset, size_t count);
/* Backend::attention (backend.rs:54-62) over contiguous K / V caches: not supported, returns
 * FHIP_ERR_BACKEND ("... not supported by this backend"), as the reference's optional methods
 * do on backends without them (backend.rs:74-88). */
int fhip_attention(fhip_backend* b, const fhip_tensor* q, const fhip_tensor* k_cache,
                   const fhip_tensor* v_cache, size_t num_kv_heads, size_t start_pos,
                   const fhip_tensor* out);

/* Backend::device_name / total_memory / available_memory / synchronize (backend.rs:126-135). */
const char* fhip_device_name(fhip_backend* b);
size_t fhip_total_memory(fhip_backend* b);
size_t fhip_available_memory(fhip_backend* b);
int fhip_synchronize(fhip_backend* b);

/* Backend::create_timer / start_timer / stop_timer / destroy_timer (backend.rs:138-147);
 * stop_timer synchronizes and returns elapsed milliseconds. */
int fhip_create_timer(fhip_backend* b, uint64_t* timer_id);
int fhip_start_timer(fhip_backend* b, uint64_t timer_id);
int fhip_stop_timer(fhip_backend* b, uint64_t timer_id, float* ms_out);
int fhip_destroy_timer(fhip_backend* b, uint64_t timer_id);

/* Backend::marker_push / marker_pop (backend.rs:150-153): roctx ranges when libroctx64 is
 * present, otherwise no-ops. */
void fhip_marker_push(fhip_backend* b, const char* name);
void fhip_marker_pop(fhip_backend* b);

/* Backend::turboquant_compress (backend.rs:166-178). */
int fhip_turboquant_compress(fhip_backend* b, const fhip_tensor* input, const fhip_tensor* rotation,
                             const fhip_tensor* centroids, uint8_t bits,
                             const fhip_tensor* packed_out, const fhip_tensor* norms_out);

/* Backend::attention_paged_tq (backend.rs:200-222); the four per-block tensor lists are
 * arrays of pool_len tensors indexed by physical block id. */
int fhip_attention_paged_tq(fhip_backend* b, const fhip_tensor* q, const int32_t* block_table,
                            size_t num_blocks, const fhip_tensor* k_packed,
                            const fhip_tensor* k_norms, const fhip_tensor* v_packed,
                            const fhip_tensor* v_norms, size_t pool_len,
                            const fhip_tensor* k_rotation, const fhip_tensor* v_rotation,
                            const fhip_tensor* k_centroids, const fhip_tensor* v_centroids,
                            uint8_t key_bits, uint8_t value_bits, size_t num_kv_heads,
                            size_t kv_len, size_t start_pos, const fhip_tensor* out);

/* Backend::matmul (backend.rs:25-27; cuda/src/backend.rs:75-128): out[M, N] = a[M, K] · b[N, K]^T,
 * fp16; a.shape[1] != b.shape[1] is InvalidShape. */
int fhip_matmul(fhip_backend* b, const fhip_tensor* a, const fhip_tensor* bm,
                const fhip_tensor* out);

/* Backend::attention_paged (backend.rs:74-88): q [T, qh, hd] fp16; the two per-block tensor
 * lists are arrays of pool_len [16, kvh, hd] fp16 tensors indexed by physical block id. */
int fhip_attention_paged(fhip_backend* b, const fhip_tensor* q, const int32_t* block_table,
                         size_t num_blocks, const fhip_tensor* k_blocks,
                         const fhip_tensor* v_blocks, size_t pool_len, size_t num_kv_heads,
                         size_t kv_len, size_t start_pos, const fhip_tensor* out);

/* Registered KV page pools (no counterpart in the reference, which copies the pool's block
 * addresses to a fresh device allocation on every attention call, cuda/src/backend.rs:295-315,
 * 625-671): `blocks` holds nlists lists of pool_len block tensors, list-major — (K, V) for
 * fhip_attention_paged_pool, (K packed, K norms, V packed, V norms) for
 * fhip_attention_paged_tq_pool. The addresses stay in device memory, so each call stages only
 * its block table. fhip_free refuses a tensor while a registered pool holds it. */
int fhip_page_pool_create(fhip_backend* b, const fhip_tensor* blocks, size_t nlists,
                          size_t pool_len, uint64_t* pool_out);
int fhip_page_pool_destroy(fhip_backend* b, uint64_t pool);
int fhip_attention_paged_pool(fhip_backend* b, const fhip_tensor* q, const int32_t* block_table,
                              size_t num_blocks, uint64_t pool, size_t num_kv_heads,
                              size_t kv_len, size_t start_pos, const fhip_tensor* out);
int fhip_attention_paged_tq_pool(fhip_backend* b, const fhip_tensor* q,
                                 const int32_t* block_table, size_t num_blocks, uint64_t pool,
                                 const fhip_tensor* k_rotation, const fhip_tensor* v_rotation,
                                 const fhip_tensor* k_centroids, const fhip_tensor* v_centroids,
                                 uint8_t key_bits, uint8_t value_bits, size_t num_kv_heads,
                                 size_t kv_len, size_t start_pos, const fhip_tensor* out);

/* QuantizedKvCacheManager::append_kv for one layer (quantized_paged_kv_cache.rs:404-500) over
 * a registered (K packed, K norms, V packed, V norms) pool: keys / values [N, kvh, hd] FP16 are
 * compressed with the layer's rotations and codebooks and token t is written straight into
 * slot (start_pos + t) % 16 of block block_table[(start_pos + t) / 16] (host array of
 * num_blocks ids). The reference compresses into scratch tensors and then issues four
 * copy_rows per page span. The backend keeps one TurboQuant plan per (rotation, codebook,
 * bits) for this and for fhip_turboquant_compress / fhip_tq_dequantize; writing or freeing
 * either tensor through this API drops the plan. */
int fhip_tq_append_kv(fhip_backend* b, uint64_t pool, const fhip_tensor* keys,
                      const fhip_tensor* values, const fhip_tensor* k_rotation,
                      const fhip_tensor* v_rotation, const fhip_tensor* k_centroids,
                      const fhip_tensor* v_centroids, uint8_t key_bits, uint8_t value_bits,
                      const int32_t* block_table, size_t num_blocks, size_t start_pos);

/* Decode attention of a batch over a registered TurboQuant pool in one call (the engine
 * dispatches Backend::attention_paged_tq per sequence, crates/fracture-engine/src/
 * batched.rs:145-194): q [B, qh, hd] fp16, one query per sequence at its last position;
 * sequence i attends seq_lens[i] positions through row i of block_tables (host,
 * [num_seqs, max_blocks]); seq_lens holds num_seqs entries; out [B, qh, hd] fp16. num_seqs
 * must equal B (q's first dimension): the host arrays are read only up to it. max_blocks is
 * between 1 and 65536. */
int fhip_attention_paged_tq_batched(fhip_backend* b, const fhip_tensor* q,
                                    const int32_t* block_tables, size_t num_seqs,
                                    size_t max_blocks, const uint32_t* seq_lens, uint64_t pool,
                                    const fhip_tensor* k_rotation, const fhip_tensor* v_rotation,
                                    const fhip_tensor* k_centroids,
                                    const fhip_tensor* v_centroids, uint8_t key_bits,
                                    uint8_t value_bits, size_t num_kv_heads,
                                    const fhip_tensor* out);

/* --- additive handle ops --------------------------------------------------------------- */

/* Backend::rope / Backend::embedding (backend.rs) with the positions / token ids already on
 * the device: `positions` / `token_ids` is a backend tensor (any dtype) whose first
 * 4 * num_positions (num_tokens) bytes are read as uint32 values. These are the forms a
 * captured graph can hold: the caller refreshes the tensor with fhip_copy_to_device before
 * each replay, where the reference passes a host slice per call (engine.rs:655-656). */
int fhip_rope_dev(fhip_backend* b, const fhip_tensor* q, const fhip_tensor* k,
                  const fhip_tensor* positions, size_t num_positions, size_t head_dim);
int fhip_embedding_dev(fhip_backend* b, const fhip_tensor* token_ids, size_t num_tokens,
                       const fhip_tensor* table, const fhip_tensor* out);

/* HIP graph capture of the backend's launches. The reference launches every kernel of a
 * layer's chain one at a time (engine.rs:621-706); here a run of launches is recorded once
 * and replayed with one launch. Between fhip_graph_begin and fhip_graph_end the ops of the
 * calling thread are recorded on the backend's stream instead of running; only ops whose
 * arguments are all device-resident and that never wait on the host are accepted: rmsnorm,
 * add, add_rmsnorm, silu_mul, copy_rows, fhip_rope_dev, fhip_embedding_dev. Every other op
 * (host arrays, host waits, allocation, the workspace users, matmul) returns FHIP_ERR_BACKEND
 * and records nothing. Other threads must keep off the backend during a capture. A graph
 * holds the tensors' device addresses: they must stay allocated while it exists.
 * fhip_graph_launch enqueues a replay on the backend's stream (asynchronous);
 * fhip_graph_destroy waits for the stream first. Graph ids are per backend. */
int fhip_graph_begin(fhip_backend* b);
int fhip_graph_end(fhip_backend* b, uint64_t* graph_out);
int fhip_graph_launch(fhip_backend* b, uint64_t graph);
int fhip_graph_destroy(fhip_backend* b, uint64_t graph);

/* Fused residual add + RMSNorm: residual += delta (in place), normed_out = rmsnorm(residual). */
int fhip_add_rmsnorm(fhip_backend* b, const fhip_tensor* residual, const fhip_tensor* delta,
                     const fhip_tensor* weight, double eps, const fhip_tensor* normed_out);
/* probs [rows, vocab] fp32 from logits [rows, vocab] fp32. */
int fhip_softmax_rows(fhip_backend* b, const fhip_tensor* logits, float temperature,
                      const fhip_tensor* probs);
/* Greedy tokens for each row, written to tokens_out (host, rows entries). Empty rows,
 * NaN and Inf give FHIP_ERR_GENERATION with the sampler's messages. */
int fhip_argmax_rows(fhip_backend* b, const fhip_tensor* logits, uint32_t* tokens_out,
                     size_t rows);
/* launch_turboquant_decompress through tensors: packed [N, kvh*pd] + norms [N, kvh] ->
 * out [N, kvh, hd] fp16. */
int fhip_tq_dequantize(fhip_backend* b, const fhip_tensor* packed, const fhip_tensor* norms,
                       const fhip_tensor* rotation, const fhip_tensor* centroids, uint8_t bits,
                       const fhip_tensor* out);
/* quantize + pack of fp32 y [N, kvh, hd] (or [rows, hd]) into packed [N, kvh*pd]. */
int fhip_tq_quantize_pack(fhip_backend* b, const fhip_tensor* y, const fhip_tensor* centroids,
                          uint8_t bits, const fhip_tensor* packed_out);

/* =====================================================================================
 * Measurement probes (no counterpart in the reference): the floors a launch reaches on this
 * device, timed the same way as the kernels above, for the benchmark's floor fractions.
 * ===================================================================================== */

/* An empty kernel of `grid` workgroups of 256 lanes. */
int fhip_probe_empty(int grid, fhip_stream_t stream);
/* A kernel that only moves memory: it reads bytes_each bytes of each of num_inputs (0-3)
 * device buffers and writes the XOR of them to each of num_outputs (0-2) buffers, in 16-byte
 * vectors over `grid` workgroups of 256 lanes; with no output it reads only (`sink`, 1 KiB of
 * device memory, is then written only if the XOR hits an impossible value). bytes_each is a
 * positive multiple of 16. */
int fhip_probe_stream(const void* const* inputs, int num_inputs, void* const* outputs,
                      int num_outputs, int64_t bytes_each, void* sink, int grid,
                      fhip_stream_t stream);

/* =====================================================================================
 * 3. Host-only helpers (no GPU)
 * ===================================================================================== */

/* TurboQuantConfig::packed_dim_per_head (turboquant.rs:99-101): ceil(head_dim * bits / 8). */
size_t fhip_tq_packed_dim_per_head(size_t head_dim, int bits);
/* LloydMaxCodebook::compute (turboquant.rs:186-250): 2^bits centroids and 2^bits - 1
 * boundaries for N(0, 1/dim). bits in 1..8. */
int fhip_tq_codebook(int dim, int bits, float* centroids_out, float* boundaries_out);
/* generate_rotation_matrix (turboquant.rs:306-338): d x d row-major Haar rotation. */
int fhip_tq_rotation_matrix(int d, uint64_t seed, float* out);
/* rotation_seeds (turboquant.rs:341-345). */
void fhip_tq_rotation_seeds(uint64_t base_seed, uint64_t layer, uint64_t* k_seed,
                            uint64_t* v_seed);
/* The RoPE inverse-frequency table of precompute_rope_freqs (lib.rs:133-139), hd/2 floats. */
void fhip_rope_freqs(int head_dim, double theta, float* out);

/* Library version string. */
const char* fhip_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FRACTURE_HIP_H */
