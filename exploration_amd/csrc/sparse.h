// Internal launch interface of the paged sparse top-k kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace st {

// Where the keys/values of (batch, absolute token, head) live.
// Contiguous (page_table == nullptr): base[B, n_tokens, H, D] holding tokens
// [token_offset, token_offset + n_tokens). Paged: pool[P, H, page_tokens, D]
// with logical page (token - token_offset) / page_tokens of batch b at
// page_table[b * pages_per_seq + logical page].
struct KvView {
  const void* k;
  const void* v;
  const int32_t* page_table;
  int64_t page_tokens, pages_per_seq, n_tokens, token_offset;
};

struct SparseArgs {
  const void* q;           // [B,Q,H,D]
  const int64_t* pos;      // [B,Q]
  KvView kv;
  float* scores;           // [B,Q,H,G] block scores (G = n_blocks)
  int64_t* ids;            // [B,Q,H,topk]
  float* top_scores;       // [B,Q,H,topk]
  float* log_zr;           // [B,Q,H]
  void* out;               // [B,Q,H,D] in the input dtype (float if out_f32)
  float* lse;              // [B,Q,H] or nullptr
  float* partial;          // pop partials [B*Q*H, n_chunks, DP + 2]
  int B, Q, H, D;
  int block, logb;
  int topk;
  int64_t n_blocks;        // blocks of the KV range (first = token_offset / block)
  int64_t id_base;         // global id of block 0 of the scores array
  float scale_log2;        // log2(e)/sqrt(D)
  int out_f32;             // write out as float instead of the input dtype
};

// Pop partial layout helpers shared by the ABI and the kernels.
inline int sparse_dp(int d) { return d <= 64 ? 64 : (d <= 128 ? 128 : 256); }
constexpr int kPopSlotsPerGroup = 4;  // blocks read by one workgroup
inline int64_t sparse_chunks(int topk) { return (topk + 2 + kPopSlotsPerGroup - 1) / kPopSlotsPerGroup; }

// Copy of k, v [batch, tokens, H, D] into pools [pool_pages, H, page_tokens,
// D] through a page table (range-relative token first_token + t of batch row
// b goes to page page_table[b * pages_per_seq + tok / page_tokens]).
struct PagedWrite {
  const void* k;
  const void* v;
  void* k_pool;
  void* v_pool;
  const int32_t* page_table;
  int64_t batch, tokens, first_token, page_tokens, pages_per_seq, pool_pages;
  int heads, head_dim, dtype;
  int64_t row_bytes;  // head_dim * element bytes
};

hipError_t launch_paged_write(const PagedWrite& w, hipStream_t stream);

hipError_t launch_sparse_scores(int dtype, const SparseArgs& a, hipStream_t stream);
hipError_t launch_sparse_select(int64_t rows, int64_t n_blocks, int topk, int64_t id_base,
                                const float* scores, int64_t* ids, float* top, float* log_zr,
                                hipStream_t stream);
hipError_t launch_sparse_pop(int dtype, const SparseArgs& a, hipStream_t stream);

}  // namespace st
