// Gated dense block attention, backward (gfx950).
//
// Closed-form derivative of the reference (st/ops/kernels/dense.py:89-182;
// st/ops/attention.py:105-139), with dQ and dK/dV computed by separate
// owners and no atomics:
//   delta = dO.O, rho = dO.RC - delta*PR                    (dense_bwd_pre)
//   remote key i of block j: u_i = exp(a_i - log Z_R), U_j = sum_j u,
//     P_i = u_i U_j exp(log Z_R - Z), gate_i = u_i (G_j / U_j - rho)
//   local key i: P_i = u_i = exp(a_i - Z)
//   direct_i = P_i (dO.v_i - delta), G_j = sum_{i in j} direct_i,
//   dA_i = (direct_i + [remote] gate_i) / sqrt(D)
//   dQ = dA K (dense_bwd_dq), dK = dA^T Q and dV = P^T dO (dense_bwd_dkv).
// One exp per score element; exp(a_i - s_j) = u_i / U_j and
// exp(a_i - log Z_R) = u_i come from the same u.
#include "dense.h"
#include "report.h"
#include "tile.h"

namespace st {

// ---------------------------------------------------------------------------
// delta and rho per (batch, query, head) row: one wave per row.
template <typename T>
__global__ __launch_bounds__(256) void dense_bwd_pre_kernel(DenseArgs a) {
  const int64_t rows = (int64_t)a.B * a.Q * a.H;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const T* o = reinterpret_cast<const T*>(a.out) + row * a.D;
  const T* g = reinterpret_cast<const T*>(a.dout) + row * a.D;
  const float* rc = a.rc + row * a.D;
  float dsum = 0.f, rsum = 0.f;
  for (int d = lane; d < a.D; d += 64) {
    const float gv = to_float<T>(g[d]);
    dsum += gv * to_float<T>(o[d]);
    rsum += gv * rc[d];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    dsum += __shfl_xor(dsum, off, 64);
    rsum += __shfl_xor(rsum, off, 64);
  }
  if (lane == 0) {
    a.delta[row] = dsum;
    a.rho[row] = rsum - dsum * a.pr[row];
  }
}

// Row statistics of one query row as the backward kernels use them.
struct RowStats {
  int rlim, llo, lhi;   // remote keys [0, rlim), local keys [llo, lhi]
  float base_r, base_l; // log2-domain subtrahends for remote / local exps
  float ezrz;           // exp(log Z_R - Z)
  float delta, rho;
};

__device__ __forceinline__ RowStats row_stats(const DenseArgs& a, int bi, int row, int hh) {
  RowStats r;
  r.rlim = 0; r.llo = 0; r.lhi = -1;
  r.base_r = 0.f; r.base_l = 0.f; r.ezrz = 0.f; r.delta = 0.f; r.rho = 0.f;
  if (row >= a.Q) return r;
  const int64_t p = a.pos[(int64_t)bi * a.Q + row];
  if (p < 0) return r;
  const int64_t N = a.N;
  const int64_t c = p / a.block;
  const int64_t lo = (c - 1) * a.block > 0 ? (c - 1) * a.block : 0;
  r.rlim = (int)(lo < N ? lo : N);
  r.llo = (int)lo;
  r.lhi = (int)(p < N - 1 ? p : N - 1);
  const int64_t sidx = ((int64_t)bi * a.Q + row) * a.H + hh;
  float zr = a.zr[sidx], z = a.z[sidx];
  zr = zr == kNegInf ? 0.f : zr;
  z = z == kNegInf ? 0.f : z;
  r.base_r = zr * kLog2e;
  r.base_l = z * kLog2e;
  r.ezrz = __expf(zr - z);
  r.delta = a.delta[sidx];
  r.rho = a.rho[sidx];
  return r;
}

// Elementwise gate derivative over a tile held as NST C tiles (keys x rows,
// lane = row). On entry s holds raw q.k dot products and dp the dO.v dot
// products; on exit s holds P and dp holds dA. `kb` is the absolute key of
// register 0 of subtile 0 for half 0. XSUM performs the cross-wave part of
// block sums for blocks wider than the tile (dK/dV kernel); it receives the
// per-row partial and returns the block total.
template <int NST, int LOGB, typename XSum>
__device__ __forceinline__ void gate_derivative(f32x16 (&s)[NST], f32x16 (&dp)[NST], const RowStats& rs,
                                                int kb, int half, float scale_log2, float scale,
                                                XSum&& xsum) {
  // u and masks
  unsigned remote_bits[NST];
#pragma unroll
  for (int st = 0; st < NST; ++st) {
    unsigned bits = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb + 32 * st + c_row(r, half);
      const bool remote = key < rs.rlim;
      const bool local = key >= rs.llo && key <= rs.lhi;
      const float x = s[st][r] * scale_log2;
      float u = 0.f;
      if (remote) u = fast_exp2(x - rs.base_r);
      else if (local) u = fast_exp2(x - rs.base_l);
      s[st][r] = u;
      bits |= (remote ? 1u : 0u) << r;
    }
    remote_bits[st] = bits;
  }
  float ublk[NST][8];
  if constexpr ((1 << LOGB) > 32 * NST) {
    // blocks wider than this tile: per-subtile partials, then the caller's
    // cross-wave total (only reached with NST == 1)
    block_sums<NST, 5>(s, ublk);
#pragma unroll
    for (int st = 0; st < NST; ++st) ublk[st][0] = xsum(ublk[st][0], 0);
  } else {
    block_sums<NST, LOGB>(s, ublk);
  }
  // P and direct
#pragma unroll
  for (int st = 0; st < NST; ++st)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const bool remote = (remote_bits[st] >> r) & 1u;
      const float u = s[st][r];
      const float p = remote ? u * ublk[st][blk_slot<LOGB>(r)] * rs.ezrz : u;
      s[st][r] = p;
      dp[st][r] = p * (dp[st][r] - rs.delta);
    }
  float gblk[NST][8];
  if constexpr ((1 << LOGB) > 32 * NST) {
    block_sums<NST, 5>(dp, gblk);
#pragma unroll
    for (int st = 0; st < NST; ++st) gblk[st][0] = xsum(gblk[st][0], 1);
  } else {
    block_sums<NST, LOGB>(dp, gblk);
  }
#pragma unroll
  for (int st = 0; st < NST; ++st)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const bool remote = (remote_bits[st] >> r) & 1u;
      float da = dp[st][r];
      if (remote) {
        const int j = blk_slot<LOGB>(r);
        const float ub = ublk[st][j];
        // u = P / (U_j e^{ZR-Z}); recover u from P to avoid keeping it live.
        const float coef = ub > 0.f ? gblk[st][j] / ub - rs.rho : -rs.rho;
        const float denom = ub * rs.ezrz;
        const float u = denom > 0.f ? s[st][r] / denom : 0.f;
        da += u * coef;
      }
      dp[st][r] = da * scale;
    }
}

// ---------------------------------------------------------------------------
// dQ: a workgroup owns 32*WAVES query rows of one (batch, head), loops over
// key tiles of NT keys (whole blocks).
template <typename T, int DP, int NT, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void dense_bwd_dq_kernel(DenseArgs a) {
  typedef Mma<T> M;
  typedef typename M::Frag Frag;
  constexpr int NTHREADS = WAVES * 64;
  constexpr int NST = NT / 32;
  constexpr int NDT = DP / 32;
  constexpr int NKC = DP / M::KW;
  constexpr int LDK = RowLd<T, DP>::value;
  constexpr bool T16 = sizeof(T) == 2;
  constexpr int LDT = TLd<NT>::value;
  constexpr int ROW_ELEMS = NT * LDK;
  constexpr int T_ELEMS = T16 ? DP * LDT : 0;
  // K, V (and K^T for 16-bit) side by side when they fit; otherwise one
  // buffer restaged in turn for each product.
  constexpr bool SEQ = (2 * ROW_ELEMS + T_ELEMS) * (int)sizeof(T) > 150 * 1024;
  constexpr int BUF_ELEMS = SEQ ? (ROW_ELEMS > T_ELEMS ? ROW_ELEMS : T_ELEMS) : 2 * ROW_ELEMS + T_ELEMS;
  __shared__ __attribute__((aligned(16))) T lds_buf[BUF_ELEMS];
  T* lds_k = lds_buf;
  T* lds_v = SEQ ? lds_buf : lds_buf + ROW_ELEMS;
  T* lds_kt = SEQ ? lds_buf : lds_buf + 2 * ROW_ELEMS;
  __shared__ int range[WAVES];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int qt = gridDim.x - 1 - blockIdx.x;
  const int bh = blockIdx.y, bi = bh / a.H, hh = bh % a.H;
  const int row = qt * 32 * WAVES + wave * 32 + col;
  const bool row_in = row < a.Q;
  const int64_t H = a.H, D = a.D, N = a.N;
  const RowStats rs = row_stats(a, bi, row, hh);

  {
    const int r0 = wave_max(rs.lhi >= 0 ? rs.lhi : -1);
    if (lane == 0) range[wave] = r0;
  }
  __syncthreads();
  int rg = range[0];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) rg = max(rg, range[w]);
  const int n_tiles = rg >= 0 ? rg / NT + 1 : 0;

  const T* kg = reinterpret_cast<const T*>(a.k) + ((int64_t)bi * N * H + hh) * D;
  const T* vg = reinterpret_cast<const T*>(a.v) + ((int64_t)bi * N * H + hh) * D;
  const int64_t kstride = H * D;
  const int64_t rbase = (((int64_t)bi * a.Q + (row_in ? row : 0)) * H + hh) * D;

  Frag qf[NKC], gf[NKC];
  {
    const T* qrow = reinterpret_cast<const T*>(a.q) + rbase;
    const T* grow = reinterpret_cast<const T*>(a.dout) + rbase;
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      const int d = c * M::KW + half * M::VEC;
      const bool ok = row_in && d < D;
      qf[c] = ok ? *reinterpret_cast<const Frag*>(qrow + d) : Frag{};
      gf[c] = ok ? *reinterpret_cast<const Frag*>(grow + d) : Frag{};
    }
  }

  f32x16 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc[dt] = zero16();

  for (int kt = 0; kt < n_tiles; ++kt) {
    const int kb = kt * NT;
    f32x16 s[NST], dp[NST];
    __syncthreads();
    stage_rows<T, NT, DP, LDK, NTHREADS>(lds_k, kg, kstride, kb, a.N, a.D);
    if constexpr (!SEQ) {
      stage_rows<T, NT, DP, LDK, NTHREADS>(lds_v, vg, kstride, kb, a.N, a.D);
      if constexpr (T16) stage_rows_t<T, NT, DP, LDT, NTHREADS>(lds_kt, kg, kstride, kb, a.N, a.D);
    }
    __syncthreads();
    scores_t<T, NST, NKC, LDK>(s, lds_k, qf, col, half);
    if constexpr (SEQ) {
      __syncthreads();
      stage_rows<T, NT, DP, LDK, NTHREADS>(lds_v, vg, kstride, kb, a.N, a.D);
      __syncthreads();
    }
    scores_t<T, NST, NKC, LDK>(dp, lds_v, gf, col, half);
    dispatch_logb(a.logb, [&]<int LOGB>() {
      gate_derivative<NST, LOGB>(s, dp, rs, kb, half, a.scale_log2, a.scale,
                                 [](float x, int) { return x; });
    });
    if constexpr (SEQ) {
      __syncthreads();
      if constexpr (T16) stage_rows_t<T, NT, DP, LDT, NTHREADS>(lds_kt, kg, kstride, kb, a.N, a.D);
      else stage_rows<T, NT, DP, LDK, NTHREADS>(lds_k, kg, kstride, kb, a.N, a.D);
      __syncthreads();
    }
    if constexpr (T16) accumulate_t<T, NST, NDT, LDT>(acc, dp, lds_kt, col, half);
    else accumulate_t<T, NST, NDT, LDK>(acc, dp, lds_k, col, half);
  }

  if (!row_in) return;
  T* dq = reinterpret_cast<T*>(a.dq) + rbase;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = 32 * dt + 8 * i + 4 * half;
      if (d < D) {
#pragma unroll
        for (int j = 0; j < 4; ++j) dq[d + j] = from_float<T>(acc[dt][4 * i + j]);
      }
    }
}

// ---------------------------------------------------------------------------
// dK/dV: a workgroup owns 128 keys of one (batch, head) (wave w: keys
// 32w..32w+31) and loops over query tiles of 32 rows. Scores are computed as
// S^T (lane = query row) for the gate algebra; P and dA are then transposed
// through LDS to form dV^T += dO^T P and dK^T += Q^T dA.
template <typename T, int DP>
__global__ __launch_bounds__(256) void dense_bwd_dkv_kernel(DenseArgs a) {
  typedef Mma<T> M;
  typedef typename M::Frag Frag;
  constexpr int NTHREADS = 256;
  constexpr int NKV = 128;
  constexpr int NDT = DP / 32;
  constexpr int NKC = DP / M::KW;
  constexpr bool T16 = sizeof(T) == 2;
  constexpr bool KV_REGS = T16 && DP <= 128;
  // query-tile operands for the key-side products: transposed for 16-bit
  // ([DP][32+4]), row-major for fp32 ([32][DP+4])
  constexpr int LDQT = T16 ? 32 + 8 : RowLd<T, DP>::value;
  constexpr int QT_ELEMS = T16 ? DP * LDQT : 32 * LDQT;
  // P / dA transposes per wave: [32 keys][32 rows (+pad)]
  constexpr int LDP = T16 ? 32 + 8 : 32 + 4;
  __shared__ __attribute__((aligned(16))) T lds_qt[QT_ELEMS];
  __shared__ __attribute__((aligned(16))) T lds_gt[QT_ELEMS];
  __shared__ __attribute__((aligned(16))) T lds_p[4][32 * LDP];
  __shared__ __attribute__((aligned(16))) T lds_da[4][32 * LDP];
  __shared__ float xbuf[2][4][32];
  __shared__ int skip;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int kt = gridDim.x - 1 - blockIdx.x;
  const int bh = blockIdx.y, bi = bh / a.H, hh = bh % a.H;
  const int kb = kt * NKV;
  const int kw = kb + 32 * wave;  // this wave's first key
  const int64_t H = a.H, D = a.D, N = a.N;
  const int64_t kstride = H * D;
  const T* kg = reinterpret_cast<const T*>(a.k) + ((int64_t)bi * N * H + hh) * D;
  const T* vg = reinterpret_cast<const T*>(a.v) + ((int64_t)bi * N * H + hh) * D;
  const T* qg = reinterpret_cast<const T*>(a.q) + ((int64_t)bi * a.Q * H + hh) * D;
  const T* gg = reinterpret_cast<const T*>(a.dout) + ((int64_t)bi * a.Q * H + hh) * D;

  // A-operand fragments of this wave's keys (lane = key kw + col).
  auto key_frag = [&](const T* base, int c) -> Frag {
    const int key = kw + col;
    const int d = c * M::KW + half * M::VEC;
    if (key < a.N && d < a.D) return *reinterpret_cast<const Frag*>(base + (int64_t)key * kstride + d);
    return Frag{};
  };
  Frag kf[KV_REGS ? NKC : 1], vf[KV_REGS ? NKC : 1];
  if constexpr (KV_REGS) {
#pragma unroll
    for (int c = 0; c < NKC; ++c) { kf[c] = key_frag(kg, c); vf[c] = key_frag(vg, c); }
  }

  f32x16 dk[NDT], dv[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) { dk[dt] = zero16(); dv[dt] = zero16(); }

  const int n_qtiles = (a.Q + 31) / 32;
  for (int it = 0; it < n_qtiles; ++it) {
    const int m0 = it * 32;
    const int row = m0 + col;
    // skip query tiles whose rows all end before this key tile
    __syncthreads();
    if (threadIdx.x == 0) skip = 1;
    __syncthreads();
    if (threadIdx.x < 32 && row < a.Q && a.pos[(int64_t)bi * a.Q + row] >= kb) skip = 0;
    __syncthreads();
    if (skip) continue;

    if constexpr (T16) {
      stage_rows_t<T, 32, DP, LDQT, NTHREADS>(lds_qt, qg, kstride, m0, a.Q, a.D);
      stage_rows_t<T, 32, DP, LDQT, NTHREADS>(lds_gt, gg, kstride, m0, a.Q, a.D);
    } else {
      stage_rows<T, 32, DP, LDQT, NTHREADS>(lds_qt, qg, kstride, m0, a.Q, a.D);
      stage_rows<T, 32, DP, LDQT, NTHREADS>(lds_gt, gg, kstride, m0, a.Q, a.D);
    }
    const RowStats rs = row_stats(a, bi, row, hh);
    // B-operand fragments of the query rows (lane = row).
    Frag qf[NKC], gf[NKC];
    {
      const bool ok_row = row < a.Q;
      const T* qrow = qg + (int64_t)(ok_row ? row : 0) * kstride;
      const T* grow = gg + (int64_t)(ok_row ? row : 0) * kstride;
#pragma unroll
      for (int c = 0; c < NKC; ++c) {
        const int d = c * M::KW + half * M::VEC;
        const bool ok = ok_row && d < D;
        qf[c] = ok ? *reinterpret_cast<const Frag*>(qrow + d) : Frag{};
        gf[c] = ok ? *reinterpret_cast<const Frag*>(grow + d) : Frag{};
      }
    }
    f32x16 s[1], dp[1];
    s[0] = zero16();
    dp[0] = zero16();
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      const Frag kfc = KV_REGS ? kf[KV_REGS ? c : 0] : key_frag(kg, c);
      const Frag vfc = KV_REGS ? vf[KV_REGS ? c : 0] : key_frag(vg, c);
      s[0] = M::mma(kfc, qf[c], s[0]);
      dp[0] = M::mma(vfc, gf[c], dp[0]);
    }
    // cross-wave block totals for blocks of 64 or 128 keys
    auto xsum = [&](float part, int which) -> float {
      if (half == 0) xbuf[which][wave][col] = part;
      __syncthreads();
      const int group = a.block >> 5;  // waves per block (2 or 4)
      const int w0 = wave & ~(group - 1);
      float tot = 0.f;
      for (int w = 0; w < group; ++w) tot += xbuf[which][w0 + w][col];
      return tot;
    };
    dispatch_logb(a.logb, [&]<int LOGB>() {
      gate_derivative<1, LOGB>(s, dp, rs, kw, half, a.scale_log2, a.scale, xsum);
    });
    // transpose P and dA into this wave's LDS regions: [key][row]
    T* pw = lds_p[wave];
    T* dw = lds_da[wave];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = c_row(r, half);
      pw[key * LDP + col] = from_float<T>(s[0][r]);
      dw[key * LDP + col] = from_float<T>(dp[0][r]);
    }
    __syncthreads();
    if constexpr (T16) {
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        const Frag bp = *reinterpret_cast<const Frag*>(pw + col * LDP + 16 * c2 + 8 * half);
        const Frag bd = *reinterpret_cast<const Frag*>(dw + col * LDP + 16 * c2 + 8 * half);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const Frag ag = *reinterpret_cast<const Frag*>(lds_gt + (32 * dt + col) * LDQT + 16 * c2 + 8 * half);
          const Frag aq = *reinterpret_cast<const Frag*>(lds_qt + (32 * dt + col) * LDQT + 16 * c2 + 8 * half);
          dv[dt] = M::mma(ag, bp, dv[dt]);
          dk[dt] = M::mma(aq, bd, dk[dt]);
        }
      }
    } else {
#pragma unroll
      for (int c2 = 0; c2 < 16; ++c2) {
        const int m = 2 * c2 + half;
        const float bp = pw[col * LDP + m];
        const float bd = dw[col * LDP + m];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          dv[dt] = M::mma(lds_gt[m * LDQT + 32 * dt + col], bp, dv[dt]);
          dk[dt] = M::mma(lds_qt[m * LDQT + 32 * dt + col], bd, dk[dt]);
        }
      }
    }
  }

  const int key = kw + col;
  if (key >= a.N) return;
  T* dkp = reinterpret_cast<T*>(a.dk) + ((int64_t)bi * N * H + hh) * D + (int64_t)key * kstride;
  T* dvp = reinterpret_cast<T*>(a.dv) + ((int64_t)bi * N * H + hh) * D + (int64_t)key * kstride;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = 32 * dt + 8 * i + 4 * half;
      if (d < D) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          dkp[d + j] = from_float<T>(dk[dt][4 * i + j]);
          dvp[d + j] = from_float<T>(dv[dt][4 * i + j]);
        }
      }
    }
}

template <typename T, int DP, int NT>
static hipError_t launch_bwd(const DenseArgs& a, hipStream_t stream) {
  constexpr int WAVES = 4;
  const int64_t rows = (int64_t)a.B * a.Q * a.H;
  note_launch((const void*)&dense_bwd_pre_kernel<T>,
              {"dense_bwd_pre", dtype_code<T>(), a.D, a.block, 4, a.D, 4, 0, (unsigned)((rows + 3) / 4), "rows"});
  hipLaunchKernelGGL((dense_bwd_pre_kernel<T>), dim3((rows + 3) / 4), dim3(256), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  dim3 gq((a.Q + 32 * WAVES - 1) / (32 * WAVES), a.B * a.H);
  note_launch((const void*)&dense_bwd_dq_kernel<T, DP, NT, WAVES>,
              {"dense_bwd_dq", dtype_code<T>(), DP, a.block, 32 * WAVES, NT, WAVES, 1, gq.x * gq.y * gq.z, "grid"});
  hipLaunchKernelGGL((dense_bwd_dq_kernel<T, DP, NT, WAVES>), gq, dim3(WAVES * 64), 0, stream, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  dim3 gk((a.N + 127) / 128, a.B * a.H);
  note_launch((const void*)&dense_bwd_dkv_kernel<T, DP>,
              {"dense_bwd_dkv", dtype_code<T>(), DP, a.block, 128, 32, 4, 1, gk.x * gk.y * gk.z, "grid"});
  hipLaunchKernelGGL((dense_bwd_dkv_kernel<T, DP>), gk, dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_bwd_t(const DenseArgs& a, hipStream_t stream) {
  const bool big_block = a.block > 64;
  if (a.D <= 64) return big_block ? launch_bwd<T, 64, 128>(a, stream) : launch_bwd<T, 64, 64>(a, stream);
  if (a.D <= 128) return big_block ? launch_bwd<T, 128, 128>(a, stream) : launch_bwd<T, 128, 64>(a, stream);
  return big_block ? launch_bwd<T, 256, 128>(a, stream) : launch_bwd<T, 256, 64>(a, stream);
}

hipError_t launch_dense_bwd(int dtype, const DenseArgs& a, hipStream_t stream) {
  if (a.tab) {
    // pipelined path (16-bit, head_dim 64/128; the workspace carries its
    // table; delta and rho come from its preparation kernel)
    return launch_dense_bwd_fast(dtype, a, stream);
  }
  switch (dtype) {
    case kBF16: return launch_bwd_t<bf16>(a, stream);
    case kF16: return launch_bwd_t<f16>(a, stream);
    default: return launch_bwd_t<float>(a, stream);
  }
}

}  // namespace st
