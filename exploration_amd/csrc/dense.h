// Internal launch interface of the dense gated attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace st {

enum DType { kF32 = 0, kF16 = 1, kBF16 = 2 };

struct DenseArgs {
  const void* q;          // [B,Q,H,D]
  const void* k;          // [B,N,H,D]
  const void* v;          // [B,N,H,D]
  const int64_t* pos;     // [B,Q], -1 = padding row
  const void* dout;       // [B,Q,H,D] (backward only)
  void* out;              // [B,Q,H,D] forward output (input dtype)
  float* rc;              // [B,Q,H,D] remote part of the output
  float* pr;              // [B,Q,H] remote probability mass
  float* zr;              // [B,Q,H] log Z_R (-inf: no remote block)
  float* z;               // [B,Q,H] logsumexp of all logits (-inf: padding)
  float* delta;           // [B,Q,H] dO.O (backward workspace, generic path)
  float* rho;             // [B,Q,H] dO.RC - delta*PR (backward workspace, generic path)
  void* dq;               // [B,Q,H,D]
  void* dk;               // [B,N,H,D]
  void* dv;               // [B,N,H,D]
  // pipelined backward workspace (null when the generic backward runs)
  int* lim;               // [B,Qp] last visible key of a row, -1 = none
  int* tmin;              // [B,Qp/64] min of lim over 64-row tiles
  int* tmax;              // [B,Qp/64] max of lim over 64-row tiles
  float2* tab;            // [B*H, nblk, Qp] per (key block, row): (beta, eps), or at bf16 with
                          // blocks of 32+ keys 16 bytes: bf16 terms of -beta/c2 and eps
  // long work items run as pieces whose fp32 partials a merge kernel adds
  // afterwards (each item's first piece writes its flag)
  int* q_count;           // [B*H*n_qtiles] 1 if the dQ item was split
  int* k_count;           // [B*H*n_ktiles] 1 if the dK/dV item was split
  float* q_part;          // dQ partials, [item][piece][wave][tile][register quad][lane] x 4
  float* k_part;          // dK/dV partials, same order
  int q_split, k_split;   // items with more tiles than this run in pieces
  int q_pieces;           // pieces of a split dQ item (2, or up to kMaxPieces for few items)
  int q_pair;             // dQ in pair mode (row tiles n-1-j and j share workgroups)
  int k_pair;             // dK/dV in pair mode (key tiles j and n-1-j)
  // pipelined forward: a long row tile runs as f_pieces pieces (consecutive
  // ranges of its remote key tiles, the last piece also its local tiles)
  // whose partial results dense_fwd_merge combines (fw0 null: never). Slot
  // mode splits a tile with more than f_split key tiles; pair mode (f_pair,
  // two pieces) runs row tiles n-1-j and j as one pair of workgroups with
  // equal tile counts.
  float* fw0;             // [piece < f_pieces-1][item][128 rows][D] remote means of the other pieces
  float* fw1;             // [item][128 rows][D] local mean of the last piece
  float* fstat;           // [item][128 rows][f_pieces + 1][4] per piece (max, row sum, sum of
                          // squared block sums), then the local (max, row sum)
  int* fflag;             // [item] 1 if the item was split
  int f_split;
  int f_pieces;
  int f_pair;
  int B, Q, N, H, D;
  int block, logb;
  int Qp, nblk;           // Q rounded up to 64; key blocks in whole 128-key tiles
  float scale;            // 1/sqrt(D)
  float scale_log2;       // log2(e)/sqrt(D)
};

// Each returns hipSuccess or the launch error; the arguments were validated
// by the caller (dtype, head_dim <= 256, block a power of two in [2,128]).
hipError_t launch_dense_fwd(int dtype, const DenseArgs& a, hipStream_t stream);
// Workspace of the pipelined forward (0 when the generic kernel runs): the
// split-item partials, indexed by row tile.
struct DenseFwdPlan {
  bool fast;
  int n_qtiles, pieces;
  size_t off_w1, off_stat, off_flag, total;
};

// Pieces a split work item runs as (2, 4 or 8): two when the items already
// fill the chip twice over (MI355X: 256 compute units), else four or
// kMaxPieces, so that a launch with few row tiles (a short chunk of queries
// over a long key range) still spreads over every compute unit.
constexpr int kMaxPieces = 8;
constexpr int kPlanCUs = 256;
inline int split_pieces(int64_t items) {
  if (8 * items <= kPlanCUs) return 8;
  if (4 * items <= kPlanCUs) return 4;
  return 2;
}
DenseFwdPlan dense_fwd_plan(int dtype, int64_t B, int64_t Q, int64_t N, int64_t H, int64_t D);
// Pipelined forward for 16-bit inputs with head_dim 64 or 128.
bool dense_fwd_fast_supported(int dtype, const DenseArgs& a);
hipError_t launch_dense_fwd_fast(int dtype, const DenseArgs& a, hipStream_t stream);
hipError_t launch_dense_bwd(int dtype, const DenseArgs& a, hipStream_t stream);

// Workspace of the backward: delta and rho (read by the generic path; the
// pipelined dQ kernel computes them in registers, the space stays so that
// one size formula serves both), plus the row limits, row-tile statistics,
// (beta, eps) table, split flags and partials of the pipelined path when it
// applies (16-bit, head_dim 64/128, table within its size cap).
struct DenseBwdPlan {
  bool fast;
  int Qp, nblk, n_rtiles, n_qtiles, n_ktiles, q_pieces;
  size_t off_rho, off_lim, off_tmin, off_tmax, off_tab, off_qcnt, off_kcnt, off_qpart, off_kpart, total;
};
DenseBwdPlan dense_bwd_plan(int dtype, int64_t B, int64_t Q, int64_t N, int64_t H, int64_t D,
                            int64_t block);
hipError_t launch_dense_bwd_fast(int dtype, const DenseArgs& a, hipStream_t stream);

}  // namespace st
