/* ie_hip.h -- C ABI of the MI355X (gfx950) paged KV-cache path.
 *
 * Host code calls these entry points with device pointers, as the reference
 * engine calls its CUDA kernel launchers (src/cuda/kernels.cuh:69-102). Every
 * entry point queues its kernels on `stream` and returns at once; results are
 * ready after the stream is synchronised. Every function returns 0 on success
 * or a nonzero IE_HIP_E* code; ie_hip_last_error() then gives the message for
 * the calling thread. No exception crosses this boundary.
 *
 * Paged KV cache (reference: src/cuda/kernels.cuh:14-38). Each layer has a
 * K pool and a V pool of `num_pages` pages; a page holds 16 token rows of
 * kv_dim = n_kv_heads * head_dim elements, row-major:
 *     pool[(page * 16 + pos % 16) * kv_dim + kv_head * head_dim + d]
 * Position `pos` of sequence `seq` lives in page
 *     tables[seq * max_pages + pos / 16].
 * Elements are float32, IEEE binary16 or bfloat16 (kv_dtype); all arithmetic
 * is float32 (MFMA tiles accumulate in float32).
 */
#ifndef IE_HIP_H_
#define IE_HIP_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IE_HIP_PAGE_SIZE 16

/* KV element types. The reference has f32 and f16 (KvLayout::f16,
 * src/cuda/kernels.cuh:37); bf16 is added here. */
enum { IE_KV_F32 = 0, IE_KV_F16 = 1, IE_KV_BF16 = 2 };

/* Status codes. */
enum {
  IE_HIP_OK = 0,
  IE_HIP_EINVAL = 1,   /* bad argument or unsupported shape */
  IE_HIP_ELAUNCH = 2,  /* a HIP call or kernel launch failed */
  IE_HIP_EFULL = 3,    /* page pool exhausted ("KV cache full: no free pages") */
  IE_HIP_ERANGE = 4,   /* sequence longer than the maximum */
  IE_HIP_ESEQ = 5      /* invalid or closed sequence id */
};

/* Where each sequence's KV rows live. Passed by value, like the reference's
 * KvLayout (src/cuda/kernels.cuh:33-38), plus `num_pages`, the pool size: the
 * kernels skip (never dereference) page ids outside [0, num_pages). */
typedef struct ie_kv_layout {
  const int32_t* tables; /* device [num_sequences * max_pages] page ids */
  int32_t max_pages;     /* row stride of `tables` */
  int32_t page_size;     /* must be IE_HIP_PAGE_SIZE */
  int32_t kv_dtype;      /* IE_KV_F32 | IE_KV_F16 | IE_KV_BF16 */
  int32_t num_pages;     /* pages in each pool */
} ie_kv_layout;

/* Message for the last failed call on this thread ("" if none). */
const char* ie_hip_last_error(void);

/* Library version string and the device it was built for ("gfx950"). */
const char* ie_hip_version(void);

/* Process-wide choice of attention kernels, like the reference's kernel
 * switches (set_tensor_cores / set_tc_fp16, src/cuda/kernels.cuh:113-118):
 *   IE_HIP_IMPL_AUTO (default) -- matrix-core (MFMA) kernels wherever the
 *       shape and KV type allow them, the VALU kernels otherwise;
 *   IE_HIP_IMPL_VALU -- always the float32 VALU kernels (for comparison);
 *   IE_HIP_IMPL_MFMA -- MFMA kernels only; unsupported shapes fail with EINVAL.
 * Returns the previous setting. Not synchronised with running kernels: set it
 * before launching. */
enum { IE_HIP_IMPL_AUTO = 0, IE_HIP_IMPL_VALU = 1, IE_HIP_IMPL_MFMA = 2 };
int ie_hip_set_attention_impl(int impl);

/* Process-wide operand precision of the matrix-core prefill on f16 caches, the
 * counterpart of the reference's set_tc_fp16 (src/cuda/cuda_runner.h:31-32,
 * src/cuda/kernels.cu:1361-1372, which picks its FP16 tensor-core prompt
 * kernel when on):
 *   IE_HIP_PREFILL_SINGLE (default) -- q and P enter the matrix cores as single
 *       f16 values rounded to nearest (the reference's tensor-core rounding,
 *       src/cuda/kernels.cu:673-674,741); errors ~6e-4 at 4,000 keys;
 *   IE_HIP_PREFILL_SPLIT -- q and P split into hi + lo f16 halves, every
 *       product issued twice: float32-level scores and weights (errors ~1e-6),
 *       at twice the matrix work. bf16 caches always split.
 * Returns the previous setting. Not synchronised with running kernels. */
enum { IE_HIP_PREFILL_SINGLE = 0, IE_HIP_PREFILL_SPLIT = 1 };
int ie_hip_set_prefill_rounding(int mode);

/* Named ranges on the ROCTX timeline (rocprofv3 --marker-trace), the
 * counterpart of the reference engine's NVTX ranges
 * (src/cuda/cuda_runner.cu:22-43,349,471). Push and pop nest per thread; a
 * null name pushes nothing. */
void ie_hip_range_push(const char* name);
void ie_hip_range_pop(void);

/* ---------------------------------------------------------------- RoPE ---
 * Host-side RoPE table, computed with the host C library exactly as the
 * reference's CPU rope does (src/ops.cpp:37-48): for p < n_pos, i < head_dim/2,
 *   inv_freq[i]                    = 1 / powf(theta, float(2i) / float(head_dim))
 *   table[p*head_dim + i]          = cosf(float(p) * inv_freq[i])
 *   table[p*head_dim + head_dim/2 + i] = sinf(float(p) * inv_freq[i])
 * `table` is host memory of n_pos * head_dim floats; upload it once. Replaces
 * the device inv_freq + cosf/sinf of the reference (src/cuda/cuda_runner.cu:184-189,
 * src/cuda/kernels.cu:290-291), which cannot match the CPU bit for bit. */
int ie_hip_rope_table(float* table, int n_pos, int head_dim, float theta);

/* Fused RoPE + paged KV append. Replaces rope_and_cache
 * (src/cuda/kernels.cuh:69-74, kernels.cu:278-307,1334-1348).
 * For each row t < T at position row_pos[t] of sequence row_seq[t]:
 *   q[t] (if q != NULL) is rotated in place;
 *   k[t] is rotated and stored (rounded to kv_dtype) at (row_seq[t], row_pos[t]);
 *   v[t] is stored (rounded) at the same slot.
 * The rotation is x0' = fma(x0, c, -(x1*s)), x1' = fma(x1, c, x0*s) with c, s
 * read from `rope_table` ([table_positions, head_dim] from ie_hip_rope_table,
 * device memory): bit-identical to the reference CPU rope. Rows whose position
 * is outside [0, table_positions) or whose page is outside the pool are skipped.
 *   q: [T, n_heads*head_dim] f32 (may be NULL)   k, v: [T, n_kv_heads*head_dim] f32
 * head_dim must be 64 or 128. */
int ie_hip_rope_and_cache(float* q, const float* k, const float* v, void* k_pool, void* v_pool,
                          const float* rope_table, int table_positions, int T,
                          const int32_t* row_pos, const int32_t* row_seq, ie_kv_layout kv,
                          int n_heads, int n_kv_heads, int head_dim, hipStream_t stream);

/* ---------------------------------------------------- decode attention ---
 * Flash-decoding over pages. Replaces attention + attention_chunks
 * (src/cuda/kernels.cuh:76-99, kernels.cu:338-507,1387-1420).
 * Row t attends causally to positions 0..row_pos[t] of its sequence. Positions
 * are cut into partitions ("chunks") of `chunk_tokens` (a multiple of 16); each
 * (row, chunk) is one workgroup producing a partial softmax result, merged
 * exactly by log-sum-exp. `num_chunks` must cover the longest context the
 * launch may see (chunks past a row's position do nothing), so one launch
 * shape serves every position, as a recorded graph needs.
 *   q, out: [T, n_heads*head_dim] f32. GQA: head h reads kv head h / (n_heads/n_kv_heads).
 * Supported: head_dim 64, n_heads/n_kv_heads <= 8 (the reference's limits at
 * this head_dim), page size 16. */

/* Chunk size (tokens) for T rows of up to `max_context` tokens with a KV cache
 * of `kv_dtype`, sized for the matrix-core kernel that dtype runs on: for
 * 16-bit caches 192 where T x (chunks at max_context) reaches 4 workgroups per
 * compute unit, 64 where T x (64-token chunks) gives at most two, else 128 (the
 * kernel splits a chunk one page pair per wave itself when the grid is small,
 * with the same result); for float32 192 where that reaches 4 workgroups per
 * compute unit, else the largest of 128/64/32 that still gives two. Results
 * depend on the chunk size, so an engine that wants
 * batch-invariant results fixes it once, from its capacity (max_batch,
 * max_seq_len), as KvEngine does. Replaces the reference's fixed
 * attention_chunks(max_seq_len) sizing (src/cuda/kernels.cu:1387-1391). */
int ie_hip_attention_chunk_tokens(int T, int max_context, int kv_dtype);

/* Chunks needed to cover `context_tokens` positions: ceil(context/chunk). */
int ie_hip_attention_chunks(int context_tokens, int chunk_tokens);

/* Bytes of workspace ie_hip_attention needs for T rows and num_chunks chunks
 * (the reference's part_o + part_ml scratch, src/cuda/kernels.cuh:82-83).
 * Allocate it once, 16-byte aligned; it needs no initialisation, since a call
 * reads only the partials it wrote itself. Calls that overlap on one
 * workspace race. */
size_t ie_hip_attention_workspace_bytes(int T, int n_heads, int head_dim, int num_chunks);

int ie_hip_attention(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                     const int32_t* row_pos, const int32_t* row_seq, ie_kv_layout kv,
                     int num_chunks, int chunk_tokens, void* workspace, int n_heads,
                     int n_kv_heads, int head_dim, hipStream_t stream);

/* ie_hip_attention without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. The
 * split-K partials go to a fixed device array of IE_HIP_NOALLOC_SCRATCH_BYTES
 * that the library holds on every GPU it runs on until the process ends; a
 * call needing more (ie_hip_attention_workspace_bytes(T, n_heads, head_dim,
 * num_chunks) above the limit: 64 rows x 14 heads hold up to 70 chunks) fails with
 * EINVAL and the message says so. It allocates and frees nothing. Calls that
 * overlap on one GPU share the array and race: serialise them (one stream).
 * Results are bit-identical to ie_hip_attention's. */
#define IE_HIP_NOALLOC_SCRATCH_BYTES (16u << 20)
int ie_hip_attention_noalloc(float* out, const float* q, const void* k_pool, const void* v_pool,
                             int T, const int32_t* row_pos, const int32_t* row_seq,
                             ie_kv_layout kv, int num_chunks, int chunk_tokens, int n_heads,
                             int n_kv_heads, int head_dim, hipStream_t stream);

/* -------------------------------------------- host-planned decode work ---
 * The decode kernel's work list built on the host, from host copies of the
 * rows' positions and sequences and of the block table -- what the reference's
 * engine holds on the host anyway (CudaEngine::run stages rows_pos/rows_seq
 * and the page tables there, src/cuda/cuda_runner.cu:366-381) -- so the 16-bit
 * kernel reaches its first K/V load after one dependent load (its item: row,
 * chunk, position, sequence, the chunk's page ids) instead of three (row
 * positions, then the row's table, then K/V). No counterpart in the reference:
 * its attention_partial_kernel reads the table itself (kernels.cu:367-371).
 * Results are bit-identical to the unplanned calls.
 *
 * ie_hip_attention_plan_ints: int32 capacity of a plan for a launch of T rows
 * and num_chunks chunks of chunk_tokens (0 for invalid arguments).
 * ie_hip_attention_plan: writes the plan to HOST memory `plan` (capacity
 * plan_capacity ints) from host row_pos / row_seq [T] and the host table
 * [max_seqs * max_pages]; pages past a row's position or its table row are
 * -1, and ids outside the pool are left for the kernel to skip. Items are
 * ordered longer chunks first (the rows' full chunks, then their shorter last
 * ones), which shortens the launch's tail; the order changes no result. Copy it to the
 * device (16-byte aligned) before the launch that uses it; it must describe
 * that launch's rows, positions, chunk_tokens and num_chunks.
 * ie_hip_attention_planned / ie_hip_rope_cache_attention_planned: as
 * ie_hip_attention / ie_hip_rope_cache_attention with the device copy of the
 * plan. row_pos still goes to the merge; tables still serve the other kernels
 * (f32 and VALU caches ignore the plan) and the fused append's page slot. */
size_t ie_hip_attention_plan_ints(int T, int num_chunks, int chunk_tokens);
int ie_hip_attention_plan(int32_t* plan, size_t plan_capacity, int T, const int32_t* row_pos,
                          const int32_t* row_seq, const int32_t* tables, int max_seqs,
                          int max_pages, int num_chunks, int chunk_tokens);
int ie_hip_attention_planned(float* out, const float* q, const void* k_pool, const void* v_pool,
                             int T, const int32_t* row_pos, const int32_t* row_seq,
                             ie_kv_layout kv, int num_chunks, int chunk_tokens, void* workspace,
                             const int32_t* plan, size_t plan_capacity, int n_heads,
                             int n_kv_heads, int head_dim, hipStream_t stream);

/* ------------------------------------------ decode step in one launch ---
 * ie_hip_rope_and_cache followed by ie_hip_attention, in one launch: the
 * reference's per-layer decode sequence rope_and_cache + attention
 * (src/cuda/kernels.cuh:69-87, called at src/cuda/cuda_runner.cu:440-445),
 * without the separate append kernel. Pages and `out` are bit-identical to the
 * two calls; unlike them, q is not rotated in place (the rotation happens in
 * registers; q is only read). Requires rows of distinct sequences (no row
 * reads the position another row of the launch appends -- a decode step), a
 * 16-bit KV cache and the matrix-core decode kernel's shapes (head_dim 64,
 * n_kv_heads*64 == 128, n_heads <= 16, chunk_tokens a multiple of 64 up to
 * 1024) under IE_HIP_IMPL_AUTO or _MFMA; otherwise EINVAL: use the two calls.
 * Arguments as for those two calls; k, v, the table and the workspace must be
 * 16-byte aligned. */
int ie_hip_rope_cache_attention_supported(int kv_dtype, int n_heads, int n_kv_heads,
                                          int head_dim, int chunk_tokens);
int ie_hip_rope_cache_attention(float* out, const float* q, const float* k, const float* v,
                                void* k_pool, void* v_pool, const float* rope_table,
                                int table_positions, int T, const int32_t* row_pos,
                                const int32_t* row_seq, ie_kv_layout kv, int num_chunks,
                                int chunk_tokens, void* workspace, int n_heads, int n_kv_heads,
                                int head_dim, hipStream_t stream);
int ie_hip_rope_cache_attention_planned(float* out, const float* q, const float* k,
                                        const float* v, void* k_pool, void* v_pool,
                                        const float* rope_table, int table_positions, int T,
                                        const int32_t* row_pos, const int32_t* row_seq,
                                        ie_kv_layout kv, int num_chunks, int chunk_tokens,
                                        void* workspace, const int32_t* plan,
                                        size_t plan_capacity, int n_heads, int n_kv_heads,
                                        int head_dim, hipStream_t stream);

/* --------------------------------------------------- prefill attention ---
 * Attention for T rows that are consecutive positions of ONE sequence
 * (row_pos[t] = row_pos[0] + t), e.g. a prompt chunk already appended with
 * ie_hip_rope_and_cache. Replaces attention_prefill_supported /
 * attention_prefill (src/cuda/kernels.cuh:89-96, kernels.cu:527-776,1350-1385).
 * f16/bf16 KV: QK^T and PV tiles on MFMA in the cache's 16-bit type (split hi +
 * lo operands, float32 accumulation). f32 KV: float32 VALU tiles. No workspace. */
int ie_hip_attention_prefill_supported(int n_heads, int n_kv_heads, int head_dim);
int ie_hip_attention_prefill(float* out, const float* q, const void* k_pool, const void* v_pool,
                             int T, const int32_t* row_pos, const int32_t* row_seq,
                             ie_kv_layout kv, int n_heads, int n_kv_heads, int head_dim,
                             hipStream_t stream);

/* ie_hip_rope_and_cache followed by ie_hip_attention_prefill for a prompt
 * chunk: the reference's per-layer prompt sequence rope_and_cache +
 * attention_prefill (src/cuda/kernels.cuh:69-74,89-96, called at
 * src/cuda/cuda_runner.cu:440-445), with the rotation of q folded into the
 * prefill kernel: K and V are rotated (K) and stored by the append as there, q
 * is only read and rotated in registers as the prefill kernel loads it (the
 * same arithmetic, so pages and `out` are bit-identical to the two calls; q in
 * memory stays unrotated, and the append skips q's 2 x 3.5 KB per row). Rows
 * as for attention_prefill (consecutive positions of one sequence); 16-bit
 * caches on the matrix-core prefill kernel only (f16, bf16; head_dim 64, at most
 * 8 query heads per KV head; not under IE_HIP_IMPL_VALU), else EINVAL: use the
 * two calls. The table must be 16-byte aligned device memory. */
int ie_hip_rope_cache_attention_prefill_supported(int kv_dtype, int n_heads, int n_kv_heads,
                                                   int head_dim);
int ie_hip_rope_cache_attention_prefill(float* out, const float* q, const float* k, const float* v,
                                        void* k_pool, void* v_pool, const float* rope_table,
                                        int table_positions, int T, const int32_t* row_pos,
                                        const int32_t* row_seq, ie_kv_layout kv, int n_heads,
                                        int n_kv_heads, int head_dim, hipStream_t stream);

/* ------------------------------------------------------------- gathers ---
 * dst[r, :] = src[rows[r], :] for r < R. Replaces gather_rows
 * (src/cuda/kernels.cuh:101-102, kernels.cu:778-783,1422-1425). */
int ie_hip_gather_rows(float* dst, const float* src, const int32_t* rows, int R, int dim,
                       hipStream_t stream);

/* Block-table gather of one sequence: dst[p, :] = pool row of (seq, p) for
 * p < len, widened to float32 ([len, kv_dim]). The paged-to-contiguous copy the
 * reference's self-test makes on the host (src/cuda/cuda_runner.cu:959-964),
 * done on the device. */
int ie_hip_gather_kv(float* dst, const void* pool, ie_kv_layout kv, int seq, int len, int kv_dim,
                     hipStream_t stream);

/* -------------------------------------------- the decode step's dense ops ---
 * The ops around the paged path in the reference's per-layer enqueue
 * (src/cuda/cuda_runner.cu:427-458): embedding, rmsnorm, the q/k/v, o_proj
 * and down projections, and the fused gate/up + SiLU. Activations are f32.
 * Results agree with the reference CPU path (src/ops.cpp, src/matrix.cpp)
 * to float32 rounding of the sums (max |d| / max |ref| <= 1e-5); the
 * embedding is exact. */

/* A weight matrix in device memory, [rows, cols] row-major: BF16 bits, or
 * INT8 values with one f32 scale per row (`scale`, INT8 only). Replaces
 * DeviceMatrix (src/cuda/kernels.cuh:40-46). */
typedef struct ie_matrix {
  const void* data;
  const float* scale;
  int32_t int8;
  int32_t rows, cols;
} ie_matrix;

/* x[t, :] = E[ids[t], :] widened to f32 (times the row's scale for INT8).
 * Replaces embedding (src/cuda/kernels.cuh:48-49, kernels.cu:191-198). */
int ie_hip_embedding(float* x, const int32_t* ids, ie_matrix e, int T, hipStream_t stream);

/* y[t, :] = x[t, :] * (1 / sqrt(mean(x[t, :]^2) + eps)) * weight; y may equal
 * x. Replaces rmsnorm (src/cuda/kernels.cuh:51-53, kernels.cu:200-209). */
int ie_hip_rmsnorm(float* y, const float* x, const float* weight, int T, int dim, float eps,
                   hipStream_t stream);

/* y[t, o] (+)= (sum_k W[o, k] * x[t, k]) * scale[o] + bias[o] (scale: INT8
 * only; bias may be NULL). accumulate != 0 adds into y (the residual
 * connection). x: [T, w.cols], y: [T, w.rows]; w.cols a multiple of 8; x and
 * the weights 16-byte aligned (8 for INT8). Replaces matmul
 * (src/cuda/kernels.cuh:55-62, kernels.cu:211-241,1242-1253). */
int ie_hip_matmul(float* y, const float* x, ie_matrix w, const float* bias, int T, int accumulate,
                  hipStream_t stream);

/* The q, k and v projections in one launch: W_qkv is Wq, Wk and Wv stacked
 * ([q_dim + 2 kv_dim, cols]) and b_qkv their biases (or NULL); rows go to
 * q [T, q_dim], k [T, kv_dim] and v [T, kv_dim]. The same results as three
 * ie_hip_matmul calls (src/cuda/cuda_runner.cu:436-438); no counterpart in the
 * reference, which launches the three. */
int ie_hip_qkv_proj(float* q, float* k, float* v, const float* x, ie_matrix w_qkv,
                    const float* b_qkv, int T, int q_dim, int kv_dim, hipStream_t stream);

/* out[t, o] = silu(x[t] . Wg[o] * sg[o]) * (x[t] . Wu[o] * su[o]), silu(v) =
 * v / (1 + exp(-v)): the MLP's gate and up projections and the SwiGLU in one
 * launch. Wg and Wu of the same shape and format. Replaces gate_up_silu
 * (src/cuda/kernels.cuh:64-66). */
int ie_hip_gate_up_silu(float* out, const float* x, ie_matrix w_gate, ie_matrix w_up, int T,
                        hipStream_t stream);

/* The rmsnorm before a projection, folded into it: the same as
 * ie_hip_rmsnorm(xn, x, norm_weight, T, cols, eps) followed by ie_hip_qkv_proj
 * (or ie_hip_gate_up_silu) on xn, in one launch and without xn: y =
 * (x * norm_weight) . W^T * (1 / sqrt(mean(x^2) + eps)), the sum of squares
 * taken in an order that depends on the matrix shape only. Equal to the two
 * calls to float32 rounding (the factors are applied in another order). For
 * matrices below 16 row tiles per compute unit (the 0.5B layer's 1,152-row
 * q/k/v and 4,864-row gate/up); norm_weight [cols], 16-byte aligned. No
 * counterpart in the reference, which launches rmsnorm and then the
 * projections (src/cuda/cuda_runner.cu:436-439,449-450). */
int ie_hip_rmsnorm_qkv_proj(float* q, float* k, float* v, const float* x,
                            const float* norm_weight, float eps, ie_matrix w_qkv,
                            const float* b_qkv, int T, int q_dim, int kv_dim, hipStream_t stream);
int ie_hip_rmsnorm_gate_up_silu(float* out, const float* x, const float* norm_weight, float eps,
                                ie_matrix w_gate, ie_matrix w_up, int T, hipStream_t stream);

/* out[r] = index of the maximum of logits[r, 0..n) for r < R: the greedy
 * token of each row, with the reference CPU argmax's semantics
 * (src/sampler.cpp:26-31): the first strict maximum in index order (ties go
 * to the lowest index), NaNs never chosen, 0 when element 0 is NaN or no
 * element exceeds -inf. Replaces argmax_rows (src/cuda/kernels.cuh:106,
 * kernels.cu:785-812), which returns INT_MAX for a row of -inf. */
int ie_hip_argmax_rows(int32_t* out, const float* logits, int R, int n, hipStream_t stream);

/* ------------------------------------------------------- page allocator ---
 * The page pool / free list / page tables behind BatchRunner (reference:
 * CudaEngine ctor src/cuda/cuda_runner.cu:191-204, open/close_sequence
 * :240-252, ensure_pages :300-313, Sequence :133-137, make_batch_runner
 * :612-622). Host-only bookkeeping; not thread-safe (one engine thread owns it,
 * src/server.h:9-17). Pages are handed out LIFO from a free list initialised so
 * that page 0 goes first; closing a sequence pushes its pages back in order. */
typedef struct ie_page_pool ie_page_pool;

/* Pool of num_pages pages for up to max_batch sequences of max_seq_len tokens.
 * Returns NULL on bad arguments (see ie_hip_last_error). */
ie_page_pool* ie_pages_create(int num_pages, int max_batch, int max_seq_len);
void ie_pages_destroy(ie_page_pool* pool);

/* Lowest free sequence slot, opened empty; -1 if all slots are busy. */
int ie_pages_open_sequence(ie_page_pool* pool);
/* Frees the sequence's pages. IE_HIP_ESEQ if seq is not open. */
int ie_pages_close_sequence(ie_page_pool* pool, int seq);
/* Makes positions 0..len-1 of seq backed by pages, taking pages from the free
 * list (IE_HIP_EFULL when it runs out, IE_HIP_ERANGE past max_seq_len,
 * IE_HIP_ESEQ for a closed id). Pages taken before a failure stay with seq. */
int ie_pages_ensure(ie_page_pool* pool, int seq, int len);
/* Tokens cached for seq (advanced by the caller after a step); -1 if closed. */
int ie_pages_sequence_length(const ie_page_pool* pool, int seq);
int ie_pages_set_sequence_length(ie_page_pool* pool, int seq, int len);
/* Pages currently owned by seq, copied to out (at most cap); returns the count. */
int ie_pages_sequence_pages(const ie_page_pool* pool, int seq, int32_t* out, int cap);
int ie_pages_total_pages(const ie_page_pool* pool);
int ie_pages_free_pages(const ie_page_pool* pool);
int ie_pages_max_batch(const ie_page_pool* pool);
int ie_pages_max_seq_len(const ie_page_pool* pool);
int ie_pages_max_pages_per_seq(const ie_page_pool* pool);
/* The host page table [max_batch * max_pages_per_seq]. It starts zero-filled;
 * as in the reference, closing a sequence does not clear its old entries. */
const int32_t* ie_pages_host_tables(const ie_page_pool* pool);
/* Copies the host table to `device_tables` on `stream` if it changed since the
 * last upload (the reference's dirty flag, src/cuda/cuda_runner.cu:379-383).
 * *uploaded (if not NULL) is set to 1 when a copy was queued. The host table is
 * staged through pinned memory owned by the pool. */
int ie_pages_upload_tables(ie_page_pool* pool, int32_t* device_tables, hipStream_t stream,
                           int* uploaded);

/* Pages a sequence of `tokens` tokens needs: ceil(tokens / 16)
 * (src/cuda/cuda_runner.cu:583). */
int ie_pages_for(int tokens);

#ifdef __cplusplus
}
#endif

#endif /* IE_HIP_H_ */
