// Scatter of contiguous K/V rows into a paged pool: the cache write of an
// inference session whose K/V live in pages of `page_tokens` tokens
// ([pool_pages, H, page_tokens, D], one page of one head contiguous).
//
// Pure data movement (HBM-bound): each workgroup takes kTokens tokens of one
// batch row; its lanes walk those tokens' rows [H, D] in source order, so the
// reads are linear and every (token, head) row lands as one contiguous run of
// D elements in its page. A token's page comes from the page table once per
// element piece (the table is tiny and stays in the L2).
#include "sparse.h"

#include "report.h"

namespace st {
namespace {

constexpr int kTokens = 16;   // tokens per workgroup
constexpr int kThreads = 256;

template <typename V>
__global__ __launch_bounds__(kThreads) void paged_write_kernel(
    const V* __restrict__ k, const V* __restrict__ v, V* __restrict__ k_pool, V* __restrict__ v_pool,
    const int32_t* __restrict__ table, int64_t tokens, int heads, int row_vecs, int64_t first,
    int64_t page_tokens, int64_t pages_per_seq, int64_t pool_pages) {
  const int64_t b = blockIdx.y;
  const int64_t t0 = (int64_t)blockIdx.x * kTokens;
  const int64_t t_end = t0 + kTokens < tokens ? t0 + kTokens : tokens;
  const int per_token = heads * row_vecs;
  const int n = (int)(t_end - t0) * per_token;
  const int64_t src0 = (b * tokens + t0) * per_token;
  for (int j = threadIdx.x; j < n; j += kThreads) {
    const int tl = j / per_token;
    const int r = j - tl * per_token;
    const int h = r / row_vecs;
    const int c = r - h * row_vecs;
    const int64_t tok = first + t0 + tl;
    const int64_t page = table[b * pages_per_seq + tok / page_tokens];
    if (page < 0 || page >= pool_pages) continue;  // a bad entry writes nothing
    const int64_t dst = ((page * heads + h) * page_tokens + tok % page_tokens) * row_vecs + c;
    k_pool[dst] = k[src0 + j];
    v_pool[dst] = v[src0 + j];
  }
}

template <typename V>
hipError_t launch_t(const PagedWrite& w, hipStream_t stream) {
  const int row_vecs = (int)(w.row_bytes / sizeof(V));
  const dim3 grid((unsigned)((w.tokens + kTokens - 1) / kTokens), (unsigned)w.batch);
  hipLaunchKernelGGL(paged_write_kernel<V>, grid, dim3(kThreads), 0, stream, static_cast<const V*>(w.k),
                     static_cast<const V*>(w.v), static_cast<V*>(w.k_pool), static_cast<V*>(w.v_pool),
                     w.page_table, w.tokens, w.heads, row_vecs, w.first_token, w.page_tokens, w.pages_per_seq,
                     w.pool_pages);
  note_launch(reinterpret_cast<const void*>(&paged_write_kernel<V>),
              LaunchInfo{"paged_kv_write", w.dtype, w.head_dim, 0, kTokens, (int)sizeof(V), kThreads / 64, 1,
                         grid.x * grid.y, "grid"});
  return hipGetLastError();
}

}  // namespace

hipError_t launch_paged_write(const PagedWrite& w, hipStream_t stream) {
  // the widest piece (16, 8, 4 or 2 bytes) dividing the row length and the
  // alignment of all four arrays
  uint64_t g = (uint64_t)w.row_bytes | reinterpret_cast<uintptr_t>(w.k) | reinterpret_cast<uintptr_t>(w.v) |
               reinterpret_cast<uintptr_t>(w.k_pool) | reinterpret_cast<uintptr_t>(w.v_pool);
  if (g % 16 == 0) return launch_t<uint4>(w, stream);
  if (g % 8 == 0) return launch_t<uint2>(w, stream);
  if (g % 4 == 0) return launch_t<uint32_t>(w, stream);
  if (g % 2 == 0) return launch_t<uint16_t>(w, stream);
  return hipErrorInvalidValue;
}

}  // namespace st
