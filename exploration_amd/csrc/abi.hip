// extern "C" entry points declared in include/st_attn.h: argument checks,
// error reporting and dispatch to the kernel launchers. Nothing here
// allocates, frees or synchronises.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>

#include "../../include/st_attn.h"
#include "dense.h"
#include "sparse.h"
#include "halo.h"
#include "pad.h"
#include "report.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return ST_OK;
}

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(ST_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

bool pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

int log2i(int64_t x) {
  int r = 0;
  while ((int64_t(1) << r) < x) ++r;
  return r;
}

int check_dtype(int dtype) {
  if (dtype != ST_DTYPE_F32 && dtype != ST_DTYPE_F16 && dtype != ST_DTYPE_BF16)
    return fail(ST_EINVAL, "unknown dtype code %d", dtype);
  return ST_OK;
}

int check_envelope(int64_t head_dim, int64_t block_size) {
  if (!pow2(block_size) || block_size < 2 || block_size > 128)
    return fail(ST_EUNSUPPORTED, "block_size %lld: the fused kernels need a power of two in [2, 128]",
                (long long)block_size);
  if (head_dim < 1 || head_dim > 256)
    return fail(ST_EUNSUPPORTED, "head_dim %lld: the fused kernels need 1 <= head_dim <= 256", (long long)head_dim);
  return ST_OK;
}

int check_sizes(int64_t batch, int64_t queries, int64_t keys, int64_t heads, int64_t head_dim,
                int64_t block_size) {
  if (batch < 1 || queries < 1 || keys < 1 || heads < 1 || head_dim < 1 || block_size < 1)
    return fail(ST_EINVAL, "attention dimensions and tile sizes must be positive");
  if (queries > (int64_t(1) << 30) || keys > (int64_t(1) << 30))
    return fail(ST_EUNSUPPORTED, "queries and keys must be below 2^30");
  if (batch * heads > 65535) return fail(ST_EUNSUPPORTED, "batch*heads must be at most 65535");
  return ST_OK;
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

size_t elem_bytes(int dtype) { return dtype == ST_DTYPE_F32 ? 4 : 2; }

// Workspace of st_dense_fwd: the kernels' own (plan, at the padded head
// dimension Dp) and, when Dp != D, zero-padded copies of q, k, v and of the
// outputs out and rc.
struct FwdLayout {
  st::DenseFwdPlan plan;
  int64_t Dp;
  size_t off_q, off_k, off_v, off_out, off_rc, total;
};

FwdLayout dense_fwd_layout(int dtype, int64_t B, int64_t Q, int64_t N, int64_t H, int64_t D) {
  FwdLayout l = {};
  l.Dp = st::padded_head_dim(D);
  l.plan = st::dense_fwd_plan(dtype, B, Q, N, H, l.Dp);
  l.total = l.plan.total;
  if (l.Dp == D) return l;
  const size_t e = elem_bytes(dtype), rq = (size_t)(B * Q * H) * l.Dp, rk = (size_t)(B * N * H) * l.Dp;
  size_t o = align256(l.total);
  l.off_q = o; o += align256(rq * e);
  l.off_k = o; o += align256(rk * e);
  l.off_v = o; o += align256(rk * e);
  l.off_out = o; o += align256(rq * e);
  l.off_rc = o; o += align256(rq * 4);
  l.total = o;
  return l;
}

// Workspace of st_dense_bwd: the kernels' own and, when Dp != D, padded
// copies of q, k, v, out, dout, rc and of the gradients.
struct BwdLayout {
  st::DenseBwdPlan plan;
  int64_t Dp;
  size_t off_q, off_k, off_v, off_out, off_dout, off_rc, off_dq, off_dk, off_dv, total;
};

BwdLayout dense_bwd_layout(int dtype, int64_t B, int64_t Q, int64_t N, int64_t H, int64_t D, int64_t b) {
  BwdLayout l = {};
  l.Dp = st::padded_head_dim(D);
  l.plan = st::dense_bwd_plan(dtype, B, Q, N, H, l.Dp, b);
  l.total = l.plan.total;
  if (l.Dp == D) return l;
  const size_t e = elem_bytes(dtype), rq = (size_t)(B * Q * H) * l.Dp, rk = (size_t)(B * N * H) * l.Dp;
  size_t o = align256(l.total);
  l.off_q = o; o += align256(rq * e);
  l.off_k = o; o += align256(rk * e);
  l.off_v = o; o += align256(rk * e);
  l.off_out = o; o += align256(rq * e);
  l.off_dout = o; o += align256(rq * e);
  l.off_rc = o; o += align256(rq * 4);
  l.off_dq = o; o += align256(rq * e);
  l.off_dk = o; o += align256(rk * e);
  l.off_dv = o; o += align256(rk * e);
  l.total = o;
  return l;
}

}  // namespace

extern "C" {

int st_abi_version(void) { return ST_ABI_VERSION; }

size_t st_launch_report(char* buf, size_t cap) { return st::report_json(buf, cap); }

const char* st_last_error(void) { return g_last_error.c_str(); }

int st_dense_supported(int dtype, int64_t head_dim, int64_t block_size) {
  if (check_dtype(dtype) != ST_OK) return 0;
  return check_envelope(head_dim, block_size) == ST_OK ? 1 : 0;
}

size_t st_dense_fwd_workspace_bytes(int dtype, int64_t batch, int64_t queries, int64_t keys,
                                    int64_t heads, int64_t head_dim, int64_t block_size) {
  if (check_dtype(dtype) || check_sizes(batch, queries, keys, heads, head_dim, block_size) ||
      check_envelope(head_dim, block_size))
    return 0;
  return dense_fwd_layout(dtype, batch, queries, keys, heads, head_dim).total;
}

int st_dense_fwd(int dtype, int64_t batch, int64_t queries, int64_t keys, int64_t heads,
                 int64_t head_dim, int64_t block_size, const void* q, const void* k,
                 const void* v, const int64_t* positions, void* out, float* rc, float* pr,
                 float* zr, float* z, void* workspace, size_t workspace_bytes, void* stream) {
  int e;
  if ((e = check_dtype(dtype)) || (e = check_sizes(batch, queries, keys, heads, head_dim, block_size)) ||
      (e = check_envelope(head_dim, block_size)))
    return e;
  if (!q || !k || !v || !positions || !out || !rc || !pr || !zr || !z)
    return fail(ST_EINVAL, "st_dense_fwd: null pointer argument");
  const FwdLayout lay = dense_fwd_layout(dtype, batch, queries, keys, heads, head_dim);
  const st::DenseFwdPlan& plan = lay.plan;
  if (workspace_bytes < lay.total || (lay.total && !workspace))
    return fail(ST_EINVAL, "st_dense_fwd: workspace of %zu bytes, %zu needed", workspace_bytes, lay.total);
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
    return fail(ST_EINVAL, "st_dense_fwd: workspace must be 256-byte aligned");
  hipStream_t s = as_stream(stream);
  char* ws = reinterpret_cast<char*>(workspace);
  const bool padded = lay.Dp != head_dim;
  const int D = (int)head_dim, Dp = (int)lay.Dp, eb = (int)elem_bytes(dtype);
  const int64_t rq = batch * queries * heads, rk = batch * keys * heads;
  st::DenseArgs a = {};
  a.q = q; a.k = k; a.v = v; a.pos = positions;
  a.out = out; a.rc = rc; a.pr = pr; a.zr = zr; a.z = z;
  if (padded) {
    hipError_t he;
    if ((he = st::launch_pad_rows(eb, ws + lay.off_q, q, rq, D, Dp, false, s)) != hipSuccess ||
        (he = st::launch_pad_rows(eb, ws + lay.off_k, k, rk, D, Dp, false, s)) != hipSuccess ||
        (he = st::launch_pad_rows(eb, ws + lay.off_v, v, rk, D, Dp, false, s)) != hipSuccess)
      return launched(he, "st_dense_fwd (pad)");
    a.q = ws + lay.off_q; a.k = ws + lay.off_k; a.v = ws + lay.off_v;
    a.out = ws + lay.off_out; a.rc = reinterpret_cast<float*>(ws + lay.off_rc);
  }
  if (plan.total) {
    a.fw0 = reinterpret_cast<float*>(ws);
    a.fw1 = reinterpret_cast<float*>(ws + plan.off_w1);
    a.fstat = reinterpret_cast<float*>(ws + plan.off_stat);
    a.fflag = reinterpret_cast<int*>(ws + plan.off_flag);
    // a row tile longer than half the longest possible one runs as two
    // pieces; with few row tiles, every tile of two or more key tiles runs
    // as plan.pieces pieces
    a.f_pieces = plan.pieces;
    a.f_split = plan.pieces > 2 ? 1 : (int)((keys + 127) / 128 + 1) / 2;
  }
  a.B = (int)batch; a.Q = (int)queries; a.N = (int)keys; a.H = (int)heads; a.D = Dp;
  a.block = (int)block_size; a.logb = log2i(block_size);
  a.scale = 1.f / sqrtf((float)head_dim);
  a.scale_log2 = a.scale * 1.4426950408889634f;
  hipError_t he = st::launch_dense_fwd(dtype, a, s);
  if (he != hipSuccess || !padded) return launched(he, "st_dense_fwd");
  if ((he = st::launch_pad_rows(eb, out, a.out, rq, D, Dp, true, s)) != hipSuccess ||
      (he = st::launch_pad_rows(4, rc, a.rc, rq, D, Dp, true, s)) != hipSuccess)
    return launched(he, "st_dense_fwd (unpad)");
  return ok();
}

size_t st_dense_bwd_workspace_bytes(int dtype, int64_t batch, int64_t queries, int64_t keys,
                                    int64_t heads, int64_t head_dim, int64_t block_size) {
  if (check_dtype(dtype) || check_sizes(batch, queries, keys, heads, head_dim, block_size) ||
      check_envelope(head_dim, block_size))
    return 0;
  return dense_bwd_layout(dtype, batch, queries, keys, heads, head_dim, block_size).total;
}

int st_dense_bwd(int dtype, int64_t batch, int64_t queries, int64_t keys, int64_t heads,
                 int64_t head_dim, int64_t block_size, const void* q, const void* k,
                 const void* v, const int64_t* positions, const void* out, const float* rc,
                 const float* pr, const float* zr, const float* z, const void* dout, void* dq,
                 void* dk, void* dv, void* workspace, size_t workspace_bytes, void* stream) {
  int e;
  if ((e = check_dtype(dtype)) || (e = check_sizes(batch, queries, keys, heads, head_dim, block_size)) ||
      (e = check_envelope(head_dim, block_size)))
    return e;
  if (!q || !k || !v || !positions || !out || !rc || !pr || !zr || !z || !dout || !dq || !dk || !dv ||
      !workspace)
    return fail(ST_EINVAL, "st_dense_bwd: null pointer argument");
  const BwdLayout lay = dense_bwd_layout(dtype, batch, queries, keys, heads, head_dim, block_size);
  const st::DenseBwdPlan& plan = lay.plan;
  if (workspace_bytes < lay.total)
    return fail(ST_EINVAL, "st_dense_bwd: workspace of %zu bytes, %zu needed", workspace_bytes, lay.total);
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
    return fail(ST_EINVAL, "st_dense_bwd: workspace must be 256-byte aligned");
  hipStream_t s = as_stream(stream);
  char* ws = reinterpret_cast<char*>(workspace);
  const bool padded = lay.Dp != head_dim;
  const int D = (int)head_dim, Dp = (int)lay.Dp, eb = (int)elem_bytes(dtype);
  const int64_t rq = batch * queries * heads, rk = batch * keys * heads;
  st::DenseArgs a = {};
  a.q = q; a.k = k; a.v = v; a.pos = positions; a.dout = dout;
  a.out = const_cast<void*>(out);
  a.rc = const_cast<float*>(rc); a.pr = const_cast<float*>(pr);
  a.zr = const_cast<float*>(zr); a.z = const_cast<float*>(z);
  a.dq = dq; a.dk = dk; a.dv = dv;
  if (padded) {
    hipError_t he;
    if ((he = st::launch_pad_rows(eb, ws + lay.off_q, q, rq, D, Dp, false, s)) != hipSuccess ||
        (he = st::launch_pad_rows(eb, ws + lay.off_k, k, rk, D, Dp, false, s)) != hipSuccess ||
        (he = st::launch_pad_rows(eb, ws + lay.off_v, v, rk, D, Dp, false, s)) != hipSuccess ||
        (he = st::launch_pad_rows(eb, ws + lay.off_out, out, rq, D, Dp, false, s)) != hipSuccess ||
        (he = st::launch_pad_rows(eb, ws + lay.off_dout, dout, rq, D, Dp, false, s)) != hipSuccess ||
        (he = st::launch_pad_rows(4, ws + lay.off_rc, rc, rq, D, Dp, false, s)) != hipSuccess)
      return launched(he, "st_dense_bwd (pad)");
    a.q = ws + lay.off_q; a.k = ws + lay.off_k; a.v = ws + lay.off_v;
    a.out = ws + lay.off_out; a.dout = ws + lay.off_dout; a.rc = reinterpret_cast<float*>(ws + lay.off_rc);
    a.dq = ws + lay.off_dq; a.dk = ws + lay.off_dk; a.dv = ws + lay.off_dv;
  }
  a.delta = reinterpret_cast<float*>(ws);
  a.rho = reinterpret_cast<float*>(ws + plan.off_rho);
  if (plan.fast) {
    a.lim = reinterpret_cast<int*>(ws + plan.off_lim);
    a.tmin = reinterpret_cast<int*>(ws + plan.off_tmin);
    a.tmax = reinterpret_cast<int*>(ws + plan.off_tmax);
    a.tab = reinterpret_cast<float2*>(ws + plan.off_tab);
    a.q_count = reinterpret_cast<int*>(ws + plan.off_qcnt);
    a.k_count = reinterpret_cast<int*>(ws + plan.off_kcnt);
    a.q_part = reinterpret_cast<float*>(ws + plan.off_qpart);
    a.k_part = reinterpret_cast<float*>(ws + plan.off_kpart);
    // an item longer than half the longest possible one runs as two pieces;
    // with few row tiles, every dQ item of two or more key tiles runs as
    // plan.q_pieces pieces
    a.q_pieces = plan.q_pieces;
    a.q_split = plan.q_pieces > 2 ? 1 : (plan.n_ktiles + 1) / 2;
    a.k_split = (plan.n_rtiles + 1) / 2;
    a.Qp = plan.Qp;
    a.nblk = plan.nblk;
  }
  a.B = (int)batch; a.Q = (int)queries; a.N = (int)keys; a.H = (int)heads; a.D = Dp;
  a.block = (int)block_size; a.logb = log2i(block_size);
  a.scale = 1.f / sqrtf((float)head_dim);
  a.scale_log2 = a.scale * 1.4426950408889634f;
  hipError_t he = st::launch_dense_bwd(dtype, a, s);
  if (he != hipSuccess || !padded) return launched(he, "st_dense_bwd");
  if ((he = st::launch_pad_rows(eb, dq, a.dq, rq, D, Dp, true, s)) != hipSuccess ||
      (he = st::launch_pad_rows(eb, dk, a.dk, rk, D, Dp, true, s)) != hipSuccess ||
      (he = st::launch_pad_rows(eb, dv, a.dv, rk, D, Dp, true, s)) != hipSuccess)
    return launched(he, "st_dense_bwd (unpad)");
  return ok();
}

// ---------------------------------------------------------------------------
// sparse

static int check_kv(const char* who, int64_t block_size, const void* k, const int32_t* page_table,
                    int64_t page_tokens, int64_t pages_per_seq, int64_t n_tokens, int64_t token_offset) {
  if (!k) return fail(ST_EINVAL, "%s: null key pointer", who);
  if (n_tokens < 1) return fail(ST_EINVAL, "%s: n_tokens must be positive", who);
  if (n_tokens >= (int64_t(1) << 31)) return fail(ST_EUNSUPPORTED, "%s: n_tokens must be below 2^31", who);
  if (token_offset < 0 || token_offset % block_size != 0)
    return fail(ST_EINVAL, "%s: cache pages/offset must be block aligned", who);
  if (page_table) {
    if (page_tokens < block_size || page_tokens % block_size != 0)
      return fail(ST_EINVAL, "%s: cache pages/offset must be block aligned", who);
    if (pages_per_seq * page_tokens < n_tokens)
      return fail(ST_EINVAL, "%s: page table covers %lld tokens, %lld needed", who,
                  (long long)(pages_per_seq * page_tokens), (long long)n_tokens);
  }
  return ST_OK;
}

static void fill_sparse(st::SparseArgs& a, int64_t batch, int64_t queries, int64_t heads,
                        int64_t head_dim, int64_t block_size, const void* q, const int64_t* positions,
                        const void* k, const void* v, const int32_t* page_table, int64_t page_tokens,
                        int64_t pages_per_seq, int64_t n_tokens, int64_t token_offset) {
  a = st::SparseArgs{};
  a.q = q; a.pos = positions;
  a.kv.k = k; a.kv.v = v; a.kv.page_table = page_table; a.kv.page_tokens = page_tokens;
  a.kv.pages_per_seq = pages_per_seq; a.kv.n_tokens = n_tokens; a.kv.token_offset = token_offset;
  a.B = (int)batch; a.Q = (int)queries; a.H = (int)heads; a.D = (int)head_dim;
  a.block = (int)block_size; a.logb = log2i(block_size);
  a.n_blocks = (n_tokens + block_size - 1) / block_size;
  a.id_base = token_offset / block_size;
  a.scale_log2 = 1.4426950408889634f / sqrtf((float)head_dim);
}

int st_sparse_scores(int dtype, int64_t batch, int64_t queries, int64_t heads, int64_t head_dim,
                     int64_t block_size, const void* q, const int64_t* positions, const void* k,
                     const int32_t* page_table, int64_t page_tokens, int64_t pages_per_seq,
                     int64_t n_tokens, int64_t token_offset, float* scores, int64_t n_blocks,
                     void* stream) {
  int e;
  if ((e = check_dtype(dtype)) || (e = check_sizes(batch, queries, 1, heads, head_dim, block_size)) ||
      (e = check_envelope(head_dim, block_size)) ||
      (e = check_kv("st_sparse_scores", block_size, k, page_table, page_tokens, pages_per_seq, n_tokens,
                    token_offset)))
    return e;
  if (!q || !positions || !scores) return fail(ST_EINVAL, "st_sparse_scores: null pointer argument");
  st::SparseArgs a;
  fill_sparse(a, batch, queries, heads, head_dim, block_size, q, positions, k, nullptr, page_table,
              page_tokens, pages_per_seq, n_tokens, token_offset);
  if (n_blocks != a.n_blocks)
    return fail(ST_EINVAL, "st_sparse_scores: n_blocks %lld, the KV range holds %lld", (long long)n_blocks,
                (long long)a.n_blocks);
  a.scores = scores;
  return launched(st::launch_sparse_scores(dtype, a, as_stream(stream)), "st_sparse_scores");
}

int st_sparse_select(int64_t rows, int64_t n_blocks, int64_t topk, int64_t id_base, const float* scores,
                     int64_t* ids, float* top_scores, float* log_zr, void* stream) {
  if (rows < 1 || n_blocks < 1) return fail(ST_EINVAL, "st_sparse_select: rows and n_blocks must be positive");
  if (topk < 1) return fail(ST_EINVAL, "topk positive; cache pages/offset must be block aligned");
  if (topk > 4096) return fail(ST_EUNSUPPORTED, "st_sparse_select: topk above 4096");
  if (n_blocks >= (int64_t(1) << 31)) return fail(ST_EUNSUPPORTED, "st_sparse_select: too many blocks");
  if (!scores || !ids || !top_scores || !log_zr) return fail(ST_EINVAL, "st_sparse_select: null pointer");
  return launched(st::launch_sparse_select(rows, n_blocks, (int)topk, id_base, scores, ids, top_scores,
                                           log_zr, as_stream(stream)),
                  "st_sparse_select");
}

size_t st_sparse_workspace_bytes(int64_t batch, int64_t queries, int64_t heads, int64_t head_dim,
                                 int64_t topk, int64_t n_blocks) {
  const size_t rows = (size_t)batch * queries * heads;
  const size_t scores = align256(sizeof(float) * rows * (size_t)n_blocks);
  const size_t partial =
      align256(sizeof(float) * rows * (size_t)st::sparse_chunks((int)topk) * (st::sparse_dp((int)head_dim) + 2));
  return scores + partial;
}

int st_sparse_pop(int dtype, int64_t batch, int64_t queries, int64_t heads, int64_t head_dim,
                  int64_t block_size, const void* q, const int64_t* positions, const void* k,
                  const void* v, const int32_t* page_table, int64_t page_tokens,
                  int64_t pages_per_seq, int64_t n_tokens, int64_t token_offset,
                  const int64_t* ids, const float* top_scores, const float* log_zr, int64_t topk,
                  int out_dtype, void* out, float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  int e;
  if (out_dtype != dtype && out_dtype != ST_DTYPE_F32)
    return fail(ST_EINVAL, "st_sparse_pop: out_dtype must be the input dtype or ST_DTYPE_F32");
  if ((e = check_dtype(dtype)) || (e = check_sizes(batch, queries, 1, heads, head_dim, block_size)) ||
      (e = check_envelope(head_dim, block_size)) ||
      (e = check_kv("st_sparse_pop", block_size, k, page_table, page_tokens, pages_per_seq, n_tokens,
                    token_offset)))
    return e;
  if (topk < 1) return fail(ST_EINVAL, "topk positive; cache pages/offset must be block aligned");
  if (topk > 4096) return fail(ST_EUNSUPPORTED, "st_sparse_pop: topk above 4096");
  if (!q || !positions || !v || !ids || !top_scores || !log_zr || !out || !workspace)
    return fail(ST_EINVAL, "st_sparse_pop: null pointer argument");
  const size_t rows = (size_t)batch * queries * heads;
  const size_t need =
      align256(sizeof(float) * rows * (size_t)st::sparse_chunks((int)topk) * (st::sparse_dp((int)head_dim) + 2));
  if (workspace_bytes < need)
    return fail(ST_EINVAL, "st_sparse_pop: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  st::SparseArgs a;
  fill_sparse(a, batch, queries, heads, head_dim, block_size, q, positions, k, v, page_table, page_tokens,
              pages_per_seq, n_tokens, token_offset);
  a.ids = const_cast<int64_t*>(ids);
  a.top_scores = const_cast<float*>(top_scores);
  a.log_zr = const_cast<float*>(log_zr);
  a.topk = (int)topk;
  a.out = out;
  a.out_f32 = out_dtype == ST_DTYPE_F32 && dtype != ST_DTYPE_F32;
  a.lse = lse;
  a.partial = reinterpret_cast<float*>(workspace);
  return launched(st::launch_sparse_pop(dtype, a, as_stream(stream)), "st_sparse_pop");
}

int st_sparse_fwd(int dtype, int64_t batch, int64_t queries, int64_t heads, int64_t head_dim,
                  int64_t block_size, int64_t topk, const void* q, const int64_t* positions,
                  const void* k, const void* v, const int32_t* page_table, int64_t page_tokens,
                  int64_t pages_per_seq, int64_t n_tokens, int64_t token_offset, void* out,
                  int64_t* ids, float* top_scores, float* log_zr, float* lse, void* workspace,
                  size_t workspace_bytes, void* stream) {
  int e;
  if ((e = check_dtype(dtype)) || (e = check_sizes(batch, queries, 1, heads, head_dim, block_size)) ||
      (e = check_envelope(head_dim, block_size)) ||
      (e = check_kv("st_sparse_fwd", block_size, k, page_table, page_tokens, pages_per_seq, n_tokens,
                    token_offset)))
    return e;
  if (topk < 1) return fail(ST_EINVAL, "topk positive; cache pages/offset must be block aligned");
  if (topk > 4096) return fail(ST_EUNSUPPORTED, "st_sparse_fwd: topk above 4096");
  if (!q || !positions || !v || !ids || !top_scores || !log_zr || !out || !workspace)
    return fail(ST_EINVAL, "st_sparse_fwd: null pointer argument");
  st::SparseArgs a;
  fill_sparse(a, batch, queries, heads, head_dim, block_size, q, positions, k, v, page_table, page_tokens,
              pages_per_seq, n_tokens, token_offset);
  const size_t need = st_sparse_workspace_bytes(batch, queries, heads, head_dim, topk, a.n_blocks);
  if (workspace_bytes < need)
    return fail(ST_EINVAL, "st_sparse_fwd: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
    return fail(ST_EINVAL, "st_sparse_fwd: workspace must be 256-byte aligned");
  const size_t rows = (size_t)batch * queries * heads;
  a.scores = reinterpret_cast<float*>(workspace);
  a.partial = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) +
                                       align256(sizeof(float) * rows * (size_t)a.n_blocks));
  a.ids = ids;
  a.top_scores = top_scores;
  a.log_zr = log_zr;
  a.topk = (int)topk;
  a.out = out;
  a.lse = lse;
  hipStream_t s = as_stream(stream);
  hipError_t he = st::launch_sparse_scores(dtype, a, s);
  if (he != hipSuccess) return launched(he, "st_sparse_fwd (scores)");
  he = st::launch_sparse_select((int64_t)rows, a.n_blocks, a.topk, a.id_base, a.scores, ids, top_scores,
                                log_zr, s);
  if (he != hipSuccess) return launched(he, "st_sparse_fwd (select)");
  return launched(st::launch_sparse_pop(dtype, a, s), "st_sparse_fwd (pop)");
}

}  // extern "C"

// ---------------------------------------------------------------------------
// paged KV cache write

int st_paged_kv_write(int dtype, int64_t batch, int64_t tokens, int64_t heads, int64_t head_dim,
                      const void* k, const void* v, const int32_t* page_table, int64_t page_tokens,
                      int64_t pages_per_seq, int64_t first_token, void* k_pool, void* v_pool,
                      int64_t pool_pages, void* stream) {
  if (int r = check_dtype(dtype)) return r;
  if (batch < 1 || tokens < 1 || heads < 1 || head_dim < 1 || page_tokens < 1 || pages_per_seq < 1 ||
      pool_pages < 1)
    return fail(ST_EINVAL, "st_paged_kv_write: dimensions must be positive");
  if (first_token < 0 || first_token + tokens > pages_per_seq * page_tokens)
    return fail(ST_EINVAL, "KV write outside owned shard");
  if (batch > 65535 || heads * head_dim > (int64_t(1) << 24))
    return fail(ST_EUNSUPPORTED, "st_paged_kv_write: batch above 65535 or heads*head_dim above 2^24");
  if (!k || !v || !page_table || !k_pool || !v_pool) return fail(ST_EINVAL, "st_paged_kv_write: null pointer");
  st::PagedWrite w{};
  w.k = k; w.v = v; w.k_pool = k_pool; w.v_pool = v_pool; w.page_table = page_table;
  w.batch = batch; w.tokens = tokens; w.first_token = first_token; w.page_tokens = page_tokens;
  w.pages_per_seq = pages_per_seq; w.pool_pages = pool_pages;
  w.heads = (int)heads; w.head_dim = (int)head_dim; w.dtype = dtype;
  w.row_bytes = head_dim * (dtype == ST_DTYPE_F32 ? 4 : 2);
  return launched(st::launch_paged_write(w, as_stream(stream)), "st_paged_kv_write");
}

// local-block window attention

static int fill_halo(st::HaloArgs& a, const char* who, int dtype, int64_t batch, int64_t groups, int64_t block_size,
                     int64_t heads, int64_t head_dim, int64_t n, int64_t start, int64_t first_key, const void* qkv,
                     const float* cos_t, const float* sin_t) {
  if (int r = check_dtype(dtype)) return r;
  if (batch < 1 || groups < 1 || block_size < 1 || heads < 1 || head_dim < 2 || n < 1)
    return fail(ST_EINVAL, "%s: dimensions must be positive", who);
  if (n > groups * block_size || n <= (groups - 1) * block_size)
    return fail(ST_EINVAL, "%s: n = %lld rows need ceil(n / block_size) = groups blocks", who, (long long)n);
  if (!st::halo_supported((int)block_size, (int)head_dim))
    return fail(ST_EUNSUPPORTED, "%s: no kernel for block_size %lld, head_dim %lld", who, (long long)block_size,
                (long long)head_dim);
  if (batch * (groups + 1) * heads >= (int64_t(1) << 31) || start < 0 || first_key < 0 || first_key > start)
    return fail(ST_EINVAL, "%s: grid or positions out of range", who);
  if (!qkv || !cos_t || !sin_t) return fail(ST_EINVAL, "%s: null pointer", who);
  a = st::HaloArgs{};
  a.B = (int)batch; a.G = (int)groups; a.b = (int)block_size; a.H = (int)heads; a.hd = (int)head_dim;
  a.n = (int)n; a.start = start; a.first_key = first_key;
  a.scale = 1.f / sqrtf((float)head_dim);
  a.qkv = qkv; a.cos_t = cos_t; a.sin_t = sin_t;
  return ST_OK;
}

int st_halo_supported(int dtype, int64_t block_size, int64_t head_dim) {
  return (dtype == ST_DTYPE_F32 || dtype == ST_DTYPE_F16 || dtype == ST_DTYPE_BF16) &&
         st::halo_supported((int)block_size, (int)head_dim);
}

int st_halo_attn_fwd(int dtype, int64_t batch, int64_t groups, int64_t block_size, int64_t heads,
                     int64_t head_dim, int64_t n, int64_t start, int64_t first_key, const void* qkv,
                     const float* cos_t, const float* sin_t, void* out, void* stream) {
  st::HaloArgs a;
  if (int r = fill_halo(a, "st_halo_attn_fwd", dtype, batch, groups, block_size, heads, head_dim, n, start,
                        first_key, qkv, cos_t, sin_t))
    return r;
  if (!out) return fail(ST_EINVAL, "st_halo_attn_fwd: null pointer");
  a.out = out;
  return launched(st::launch_halo_fwd(dtype, a, as_stream(stream)), "st_halo_attn_fwd");
}

int st_halo_attn_bwd(int dtype, int64_t batch, int64_t groups, int64_t block_size, int64_t heads,
                     int64_t head_dim, int64_t n, int64_t start, int64_t first_key, const void* qkv,
                     const float* cos_t, const float* sin_t, const void* out, const void* dout, void* dqkv,
                     void* stream) {
  st::HaloArgs a;
  if (int r = fill_halo(a, "st_halo_attn_bwd", dtype, batch, groups, block_size, heads, head_dim, n, start,
                        first_key, qkv, cos_t, sin_t))
    return r;
  if (!out || !dout || !dqkv) return fail(ST_EINVAL, "st_halo_attn_bwd: null pointer");
  a.out = const_cast<void*>(out);
  a.dout = dout;
  a.dqkv = dqkv;
  return launched(st::launch_halo_bwd(dtype, a, as_stream(stream)), "st_halo_attn_bwd");
}

// ---------------------------------------------------------------------------
// sparse forward without a caller workspace

namespace {

// The workspace of st_sparse_fwd_noalloc: the block scores of every row
// followed by the read's slot partials. One copy per GPU (the module's
// device globals), held until the process ends; every call on a GPU reuses
// and overwrites it. Host code never passes the array's name to a kernel: it
// uses the device address looked up below.
constexpr size_t kScratchBytes = ST_SPARSE_NOALLOC_SCRATCH_BYTES;
__device__ __attribute__((aligned(256))) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, null until looked up

// Device address of the current device's `scratch`, looked up once per
// device (hipGetSymbolAddress with that device current).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return launched(e, "st_sparse_fwd_noalloc (hipGetDevice)");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(ST_EUNSUPPORTED, "st_sparse_fwd_noalloc: device %d beyond the %d supported", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return launched(e, "st_sparse_fwd_noalloc (hipGetSymbolAddress)");
    if (!p) return fail(ST_ELAUNCH, "st_sparse_fwd_noalloc: no device address for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ST_OK;
}

}  // namespace

extern "C" {

size_t st_sparse_noalloc_scratch_bytes(void) { return kScratchBytes; }

int st_sparse_fwd_noalloc(int dtype, int64_t batch, int64_t queries, int64_t heads, int64_t head_dim,
                          int64_t block_size, int64_t topk, const void* q, const int64_t* positions,
                          const void* k, const void* v, const int32_t* page_table, int64_t page_tokens,
                          int64_t pages_per_seq, int64_t n_tokens, int64_t token_offset, void* out,
                          int64_t* ids, float* top_scores, float* log_zr, float* lse, void* stream) {
  int e;
  if ((e = check_dtype(dtype)) || (e = check_sizes(batch, queries, 1, heads, head_dim, block_size)) ||
      (e = check_envelope(head_dim, block_size)) ||
      (e = check_kv("st_sparse_fwd_noalloc", block_size, k, page_table, page_tokens, pages_per_seq, n_tokens,
                    token_offset)))
    return e;
  if (topk < 1) return fail(ST_EINVAL, "topk positive; cache pages/offset must be block aligned");
  const int64_t n_blocks = (n_tokens + block_size - 1) / block_size;
  const size_t need = st_sparse_workspace_bytes(batch, queries, heads, head_dim, topk, n_blocks);
  if (need > kScratchBytes)
    return fail(ST_EUNSUPPORTED,
                "st_sparse_fwd_noalloc: this problem needs %zu bytes of scratch, the built-in array holds %zu "
                "(call st_sparse_fwd with a workspace)",
                need, kScratchBytes);
  void* ws = nullptr;
  if ((e = scratch_address(&ws))) return e;
  return st_sparse_fwd(dtype, batch, queries, heads, head_dim, block_size, topk, q, positions, k, v, page_table,
                       page_tokens, pages_per_seq, n_tokens, token_offset, out, ids, top_scores, log_zr, lse, ws,
                       kScratchBytes, stream);
}

}  // extern "C"
