/*
 * st_attn.h: C ABI of the MI355X (gfx950) Stack attention kernels.
 *
 * A drop-in for the GPU kernel layer of zhjerry25/Exploration (package `st`):
 * each entry point replaces the Triton launch(es) named in its comment. All
 * tensors are device pointers to contiguous row-major arrays; the caller owns
 * every buffer (these functions never allocate, free or synchronise) and
 * passes the HIP stream to launch on (NULL = the legacy default stream).
 *
 * Return value: ST_OK, or a status whose message st_last_error() returns
 * (thread-local). ST_EINVAL and ST_EUNSUPPORTED correspond to the reference's
 * ValueError (st/ops/attention.py:155-162,171-172; st/ops/sparse.py:108-110),
 * ST_ELAUNCH to a RuntimeError carrying the HIP error string.
 *
 * Layouts (reference docs/API.md:154):
 *   q, out, rc, dout, dq    [B, Q, H, D]   element type `dtype`, rc float
 *   k, v, dk, dv            [B, N, H, D]
 *   positions               [B, Q] int64, absolute key index, -1 = padding row
 *   pr, zr, z, log_zr, lse  [B, Q, H] float
 *   block scores            [B, Q, H, G] float, G = blocks of the KV range
 *   ids / top scores        [B, Q, H, topk] int64 / float
 * Paged KV (no reference counterpart; the reference slices contiguous pages,
 * st/ops/sparse.py:75-96): pool [P, H, page_tokens, D] addressed through
 * page_table [B, pages_per_seq] int32 (logical page -> pool page).
 */
#ifndef ST_ATTN_H
#define ST_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ST_ABI_VERSION 5

#define ST_DTYPE_F32 0
#define ST_DTYPE_F16 1
#define ST_DTYPE_BF16 2

#define ST_OK 0
#define ST_EINVAL 1
#define ST_EUNSUPPORTED 2
#define ST_ELAUNCH 3

/* Version of this ABI (ST_ABI_VERSION). */
int st_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* st_last_error(void);

/* Launch records as a JSON array, one object per (kernel, device, dtype,
 * head_dim, block_size, mode) launched so far: the reference's report
 * fields (st/ops/kernels/launch.py:52-56,96-98: kernel, path, device, dtype,
 * head_dim, block_size, tile_m, tile_n, num_warps = waves per workgroup,
 * num_stages = LDS buffers per operand, shared_memory_bytes) plus vgprs,
 * scratch_bytes, workgroups and mode. Writes at most cap bytes (NUL
 * terminated) and returns the size the whole report needs. */
size_t st_launch_report(char* buf, size_t cap);

/* 1 if the fused kernels support (dtype, head_dim, block_size), else 0.
 * Replaces the Triton capability predicate triton_supported
 * (st/ops/attention.py:142-145): fp32/fp16/bf16, block a power of two in
 * [2, 128], head_dim <= 256. The reference pads D to a power of two inside
 * its kernel (st/ops/kernels/dense.py:210); here a head_dim that is not a
 * multiple of 8 runs the dense kernels on zero-padded copies held in the
 * workspace (its size includes them) and the sparse kernels with element
 * loads. */
int st_dense_supported(int dtype, int64_t head_dim, int64_t block_size);

/* Bytes of device workspace st_dense_fwd needs for this problem (0 if none
 * or if the arguments are invalid). The pipelined 16-bit path (head_dim 64
 * or 128) runs the longest causal row tiles as two pieces and merges their
 * partial results: per 128-row tile 2 x 128 x head_dim floats of partial
 * means, 128 x 8 floats of statistics and a flag. A head_dim that is not a
 * multiple of 8 adds padded copies of q, k, v, out and rc. No reference
 * counterpart:
 * the reference's Triton forward allocates its own buffers
 * (st/ops/kernels/dense.py:200-203). */
size_t st_dense_fwd_workspace_bytes(int dtype, int64_t batch, int64_t queries, int64_t keys,
                                    int64_t heads, int64_t head_dim, int64_t block_size);

/* Gated dense forward. Replaces the `_forward` launch of
 * st/ops/kernels/dense.py:197-217 (kernel st/ops/kernels/dense.py:32-86).
 * Writes out (dtype) and the saved statistics rc, pr, zr, z (float).
 * workspace: st_dense_fwd_workspace_bytes() bytes, 256-byte aligned (may be
 * NULL when that is 0). */
int st_dense_fwd(int dtype, int64_t batch, int64_t queries, int64_t keys, int64_t heads,
                 int64_t head_dim, int64_t block_size, const void* q, const void* k,
                 const void* v, const int64_t* positions, void* out, float* rc, float* pr,
                 float* zr, float* z, void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of device workspace st_dense_bwd needs for this problem (0 if the
 * arguments are invalid): per-row delta and rho, plus, on the pipelined
 * 16-bit path (head_dim 64 or 128), row limits and a per-(row, key block)
 * table of 8 bytes, B*H*ceil(Q/64)*64*ceil(N/128)*(128/block_size) entries,
 * capped at 4 GiB (larger problems take the generic kernels). No reference
 * counterpart: the reference's Triton backward allocates its own buffers
 * (st/ops/kernels/dense.py:221-233). */
size_t st_dense_bwd_workspace_bytes(int dtype, int64_t batch, int64_t queries, int64_t keys,
                                    int64_t heads, int64_t head_dim, int64_t block_size);

/* Gated dense backward (first derivatives). Replaces the `_preprocess`,
 * `_backward_q` and `_backward_kv` launches of st/ops/kernels/dense.py:221-233.
 * Inputs are the forward's inputs and saved statistics plus dout; writes
 * dq, dk, dv in `dtype`. */
int st_dense_bwd(int dtype, int64_t batch, int64_t queries, int64_t keys, int64_t heads,
                 int64_t head_dim, int64_t block_size, const void* q, const void* k,
                 const void* v, const int64_t* positions, const void* out, const float* rc,
                 const float* pr, const float* zr, const float* z, const void* dout, void* dq,
                 void* dk, void* dv, void* workspace, size_t workspace_bytes, void* stream);

/* Exact block scores s_j = logsumexp over block j of q.k/sqrt(D) for the
 * blocks [token_offset/b, token_offset/b + n_blocks) with the reference's
 * visibility mask (-inf unless j < p//b - 1 and the block lies inside the KV
 * range). Replaces block_scores / `_scores`
 * (st/ops/kernels/sparse.py:9-35,81-100). KV addressing: page_table == NULL
 * means contiguous k[B, n_tokens, H, D] holding absolute tokens
 * [token_offset, token_offset + n_tokens); otherwise the paged pool. */
int st_sparse_scores(int dtype, int64_t batch, int64_t queries, int64_t heads, int64_t head_dim,
                     int64_t block_size, const void* q, const int64_t* positions, const void* k,
                     const int32_t* page_table, int64_t page_tokens, int64_t pages_per_seq,
                     int64_t n_tokens, int64_t token_offset, float* scores, int64_t n_blocks,
                     void* stream);

/* Top-k blocks per row of scores [rows, n_blocks]: ids (block index +
 * id_base, -1 where the score is -inf) and scores in descending order, ties
 * by ascending block id, plus log_zr = logsumexp of the row. Replaces the
 * running top-k and log Z_R of st/ops/sparse.py:121-139,154. */
int st_sparse_select(int64_t rows, int64_t n_blocks, int64_t topk, int64_t id_base,
                     const float* scores, int64_t* ids, float* top_scores, float* log_zr,
                     void* stream);

/* Bytes of device workspace st_sparse_pop / st_sparse_fwd need. */
size_t st_sparse_workspace_bytes(int64_t batch, int64_t queries, int64_t heads, int64_t head_dim,
                                 int64_t topk, int64_t n_blocks);

/* Softmax read over the local window and the selected blocks, gated by
 * log_zr. Replaces sparse_pop / `_pop` and the LSE merge of
 * st/ops/kernels/sparse.py:38-78,103-113 and st/ops/sparse.py:157-162.
 * Writes out in out_dtype (`dtype`, or ST_DTYPE_F32 for the reference's
 * float32 partial, st/ops/kernels/sparse.py:108) and, if lse != NULL, the
 * row logsumexp (float). */
int st_sparse_pop(int dtype, int64_t batch, int64_t queries, int64_t heads, int64_t head_dim,
                  int64_t block_size, const void* q, const int64_t* positions, const void* k,
                  const void* v, const int32_t* page_table, int64_t page_tokens,
                  int64_t pages_per_seq, int64_t n_tokens, int64_t token_offset,
                  const int64_t* ids, const float* top_scores, const float* log_zr, int64_t topk,
                  int out_dtype, void* out, float* lse, void* workspace, size_t workspace_bytes,
                  void* stream);

/* Whole sparse forward: scores, selection and read in one call
 * (st/ops/sparse.py:99-174 on one device). ids/top_scores/log_zr receive
 * the selection; scores of all n_blocks blocks live in the workspace. */
int st_sparse_fwd(int dtype, int64_t batch, int64_t queries, int64_t heads, int64_t head_dim,
                  int64_t block_size, int64_t topk, const void* q, const int64_t* positions,
                  const void* k, const void* v, const int32_t* page_table, int64_t page_tokens,
                  int64_t pages_per_seq, int64_t n_tokens, int64_t token_offset, void* out,
                  int64_t* ids, float* top_scores, float* log_zr, float* lse, void* workspace,
                  size_t workspace_bytes, void* stream);

/* st_sparse_fwd without a caller workspace. No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * workspace is a file-scope device array of ST_SPARSE_NOALLOC_SCRATCH_BYTES
 * per GPU, held until the process ends; problems whose workspace
 * (st_sparse_workspace_bytes) exceeds it fail with ST_EUNSUPPORTED. Calls
 * that overlap on one GPU (concurrent streams or threads) share that array
 * and race: serialise them. Same arguments and results as st_sparse_fwd;
 * allocates nothing (the first call on a device looks up the array's
 * device address). */
#define ST_SPARSE_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
size_t st_sparse_noalloc_scratch_bytes(void);
int st_sparse_fwd_noalloc(int dtype, int64_t batch, int64_t queries, int64_t heads, int64_t head_dim,
                          int64_t block_size, int64_t topk, const void* q, const int64_t* positions,
                          const void* k, const void* v, const int32_t* page_table, int64_t page_tokens,
                          int64_t pages_per_seq, int64_t n_tokens, int64_t token_offset, void* out,
                          int64_t* ids, float* top_scores, float* log_zr, float* lse, void* stream);

/* Write of K and V rows k, v [batch, tokens, H, D] into a paged cache
 * k_pool, v_pool [pool_pages, H, page_tokens, D]: token t of batch row b
 * (range-relative token first_token + t) lands in pool page
 * page_table[b * pages_per_seq + (first_token + t) / page_tokens], row
 * (first_token + t) % page_tokens. page_table holds batch * pages_per_seq
 * int32 entries; an entry outside [0, pool_pages) is skipped (nothing is
 * written for its tokens), so a bad table cannot write outside the pools.
 * Replaces KVCache.write (st/runtime/inference.py:45-52), which copies into
 * a contiguous [B, N, H, D] slab; the paged pool is what st_sparse_fwd
 * reads. */
int st_paged_kv_write(int dtype, int64_t batch, int64_t tokens, int64_t heads, int64_t head_dim,
                      const void* k, const void* v, const int32_t* page_table, int64_t page_tokens,
                      int64_t pages_per_seq, int64_t first_token, void* k_pool, void* v_pool,
                      int64_t pool_pages, void* stream);

/* Two-block window attention of the model's local blocks (no st.ops
 * counterpart: the reference computes it with torch's scaled dot-product
 * attention, st/models/blocks.py:131-160, after the rotary embedding of
 * blocks.py:76-93). qkv [B, (G+1)*b, 3, H, hd] is the projection output of
 * [previous block ++ the chunk padded to G*b rows]; query block g attends to
 * raw blocks g and g+1, key kk visible to query i when kk <= i + b and its
 * absolute position lies in [first_key, start + n). cos_t / sin_t [2b, hd/2]
 * float: the rotary cos/sin of positions -b..b-1, as the reference computes
 * them and rounded to dtype. out [B, n, H, hd] (dtype) receives the first n
 * rows. 1 if (block_size, head_dim) has a kernel, else 0. */
int st_halo_supported(int dtype, int64_t block_size, int64_t head_dim);
int st_halo_attn_fwd(int dtype, int64_t batch, int64_t groups, int64_t block_size, int64_t heads,
                     int64_t head_dim, int64_t n, int64_t start, int64_t first_key, const void* qkv,
                     const float* cos_t, const float* sin_t, void* out, void* stream);
/* Backward: writes every element of dqkv (same layout as qkv) from dout
 * [B, n, H, hd] and the forward's out; deterministic (no atomics). */
int st_halo_attn_bwd(int dtype, int64_t batch, int64_t groups, int64_t block_size, int64_t heads,
                     int64_t head_dim, int64_t n, int64_t start, int64_t first_key, const void* qkv,
                     const float* cos_t, const float* sin_t, const void* out, const void* dout, void* dqkv,
                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ST_ATTN_H */
