// Gated dense block attention, backward: pipelined gfx950 path for 16-bit
// inputs with head_dim 64 or 128 (the hot shapes).
//
// Derivative (st/ops/kernels/dense.py:89-182; st/ops/attention.py:105-139):
// for a query row with statistics Z, log Z_R, delta = dO.O, rho = dO.RC -
// delta*PR and logits a_i = q.k_i/sqrt(D),
//   remote key i in block j: u_i = exp(a_i - log Z_R), U_j = sum_{i in j} u_i,
//     P_i = u_i U_j e^{log Z_R - Z},
//     dA_i = P_i (dP_i - delta) + u_i (G_j / U_j - rho),
//     G_j = sum_{i in j} P_i (dP_i - delta);
//   local key i: P_i = exp(a_i - Z), dA_i = P_i (dP_i - delta).
// Both cases have the form
//   P_i = exp2(a_i log2(e) - beta_j),  dA_i = P_i (dP_i + eps_j)
// with one (beta_j, eps_j) per (row, key block):
//   remote: beta_j = Z log2(e) - log2 U_j,
//           eps_j = (G_j / U_j - rho) / (U_j e^{log Z_R - Z}) - delta;
//   local:  beta_j = Z log2(e), eps_j = -delta;
//   beyond the row's window: beta_j = +inf (P = 0), eps_j = 0.
//
// Kernels:
//  * dense_bwd_dq_fast: lane = query row, the layout in which block sums are
//    in-lane; computes delta and rho of its rows (st/ops/kernels/dense.py:
//    89-100), recomputes S and dP, writes dQ and the (beta, eps) table, and
//    per row the last visible key, per 64-row tile its min/max (which row
//    tiles a key tile must visit, and which need masks);
//  * dense_bwd_dkv_fast: lane = key; per element one exp2 and two FMAs from
//    the table (at bf16 with blocks of 32+ keys the table's terms enter S and
//    dP through one extra MFMA each, then one multiply each), no cross-lane
//    or cross-wave reductions, dK/dV in registers.
// K/V (dQ kernel) and Q/dO (dK/dV kernel) tiles are staged with asynchronous
// global->LDS copies into swizzled, double-buffered LDS; transposed operands
// come from ds_read_tr16_b64. Workgroups are numbered head-fastest, so the
// dispatcher's round-robin over the XCDs keeps one head per XCD L2.
#include <type_traits>

#include "dense.h"
#include "report.h"
#include "tile.h"

namespace st {

namespace {

constexpr int kKT = 128;       // keys per dK/dV workgroup and per dQ key tile
// Cost, in key tiles, of splitting a dQ row tile into two pieces (the second
// workgroup's dispatch, prologue and cold first tiles, the partial's store
// and merge), and the same for a dK/dV key tile in 64-row steps. Measured on
// cfg2 (fwd+bwd step): dQ 2..9 -> 3 fastest, dK/dV 2..8 within noise.
constexpr int kQPieceCost = 3;
constexpr int kKPieceCost = 4;
constexpr int kRT = 64;        // query rows per dK/dV step / row-tile statistic
constexpr int kFewRTiles = 8;  // dK/dV launches over at most this many row tiles run unsplit
constexpr int kMaxRTiles = 2048;
constexpr size_t kMaxTable = size_t(4) << 30;
constexpr float kInf = __builtin_inff();

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace

// Table entries per (row, key block). bf16 with blocks of 32+ keys (a wave's
// 32 keys in one block): 16 bytes, -beta/c2 and eps each as three bf16
// terms (then two zeros), which the dK/dV kernel adds to S and dP by one
// MFMA each (an extra contraction chunk against constant ones), so that no
// lane reads the table's broadcast values per score. Otherwise the float2
// (beta, eps).
template <typename T, int LOGB> struct AugTable {
  static constexpr bool on = std::is_same<T, bf16>::value && LOGB >= 5;
  static constexpr int bytes = on ? 16 : 8;
};

// v as three bf16 terms: |v - t[0] - t[1] - t[2]| is at most about 2^-26 |v|
__device__ __forceinline__ void split3_bf16(float v, bf16 (&t)[3]) {
  t[0] = (bf16)v;
  const float r0 = v - (float)t[0];
  t[1] = (bf16)r0;
  t[2] = (bf16)(r0 - (float)t[1]);
}

DenseBwdPlan dense_bwd_plan(int dtype, int64_t B, int64_t Q, int64_t N, int64_t H, int64_t D,
                            int64_t block) {
  DenseBwdPlan p = {};
  const size_t rows = align256(sizeof(float) * (size_t)(B * Q * H));
  p.off_rho = rows;
  p.total = 2 * rows;
  // 32-bit buffer offsets within one batch's K/V and Q/dO
  const bool shape_ok = (dtype == kBF16 || dtype == kF16) && (D == 64 || D == 128) && block <= kKT &&
                        N * H * D * 2 < (int64_t(1) << 31) && Q * H * D * 2 < (int64_t(1) << 31);
  if (!shape_ok) return p;
  const int64_t Qp = (Q + kRT - 1) / kRT * kRT;
  const int64_t n_rtiles = Qp / kRT;
  const int64_t nblk = (N + kKT - 1) / kKT * (kKT / block);
  const size_t ent = dtype == kBF16 && block >= 32 ? 16 : sizeof(float2);  // AugTable<T, LOGB>::bytes
  const size_t tab = ent * (size_t)(B * H) * (size_t)nblk * (size_t)Qp;
  if (n_rtiles > kMaxRTiles || tab > kMaxTable) return p;
  p.fast = true;
  p.Qp = (int)Qp;
  p.nblk = (int)nblk;
  p.n_rtiles = (int)n_rtiles;
  p.off_lim = p.total;
  p.off_tmin = p.off_lim + align256(sizeof(int) * (size_t)(B * Qp));
  p.off_tmax = p.off_tmin + align256(sizeof(int) * (size_t)(B * n_rtiles));
  p.off_tab = p.off_tmax + align256(sizeof(int) * (size_t)(B * n_rtiles));
  p.n_qtiles = (int)((Q + 127) / 128);
  p.n_ktiles = (int)((N + kKT - 1) / kKT);
  const size_t q_items = (size_t)(B * H) * p.n_qtiles, k_items = (size_t)(B * H) * p.n_ktiles;
  p.off_qcnt = p.off_tab + align256(tab);
  p.off_kcnt = p.off_qcnt + align256(sizeof(int) * q_items);
  p.off_qpart = p.off_kcnt + align256(sizeof(int) * k_items);
  // per item and piece: 128 rows (keys) x D floats (x2 for dK and dV); dQ
  // items run as more than two pieces when they are few
  p.q_pieces = split_pieces((int64_t)q_items);
  p.off_kpart = p.off_qpart + align256(sizeof(float) * q_items * p.q_pieces * 128 * (size_t)D);
  p.total = p.off_kpart + align256(sizeof(float) * k_items * 2 * 2 * 128 * (size_t)D);
  return p;
}

// A piece of a split item stores its fp32 accumulators in register-quad
// order ([piece][wave][tile][quad][lane] x 4 floats: one 16-byte store per
// lane and quad, a wave's 1 KiB contiguous); dense_bwd_merge adds the
// pieces after the kernel (the item's first piece records whether it was
// split).
template <int NACC>
__device__ __forceinline__ void store_piece(const f32x16 (&acc)[NACC], float* part, int piece) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  f32x4* mine = reinterpret_cast<f32x4*>(part + ((size_t)piece * 4 + wave) * (NACC * 16 * 64));
#pragma unroll
  for (int t = 0; t < NACC; ++t)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      mine[(t * 4 + q) * 64 + lane] = f32x4{acc[t][4 * q], acc[t][4 * q + 1], acc[t][4 * q + 2], acc[t][4 * q + 3]};
}

// ---------------------------------------------------------------------------
// dQ and the (beta, eps) table. A workgroup owns 128 query rows (wave w: rows
// 32w..32w+31, lane = row) of one (batch, head) and walks the key tiles of
// its causal range. Score tiles are transposed (S^T = K Q^T, dP^T = V dO^T).
template <typename T, int DP, int LOGB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void dense_bwd_dq_fast_kernel(DenseArgs a, int n_qtiles) {
  typedef Mma<T> M;
  typedef typename M::Frag Frag;
  constexpr int WAVES = 4;
  constexpr int NT = kKT;
  constexpr int NST = NT / 32;
  constexpr int NDT = DP / 32;
  constexpr int NKC = DP / M::KW;
  constexpr int TILE = NT * DP;
  constexpr int b = 1 << LOGB;
  __shared__ __attribute__((aligned(16))) T k0s[TILE];
  __shared__ __attribute__((aligned(16))) T k1s[TILE];
  __shared__ __attribute__((aligned(16))) T v0s[TILE];
  __shared__ __attribute__((aligned(16))) T v1s[TILE];
  __shared__ int range[2][2][WAVES];  // two row tiles: this one and the pair partner
  __shared__ int lim_mm[2][WAVES];    // per wave: min and max of its rows' last visible keys

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int BH = a.B * a.H;
  const int bh = blockIdx.x % BH, slot = (int)(blockIdx.x / BH);
  const int bi = bh / a.H, hh = bh % a.H;
  const int64_t H = a.H, D = a.D, N = a.N;

  // Key tiles of row tile qt (LDS slot k): the count up to the last
  // visible key of any row, and how many lie below every row's remote limit
  // (all keys remote, no masks). row_pos loads a lane's position,
  // publish_range writes the wave's part, collect_range (after a barrier)
  // combines the waves'.
  auto row_pos = [&](int qt) -> int64_t {
    const int row = qt * 32 * WAVES + wave * 32 + col;
    return row < a.Q ? a.pos[(int64_t)bi * a.Q + row] : -1;
  };
  auto publish_range = [&](int64_t p, int k) {
    int rl = 0, lh = -1;
    if (p >= 0) {
      const int64_t c = p >> LOGB;
      const int64_t lo = (c - 1) * b > 0 ? (c - 1) * b : 0;
      rl = (int)(lo < N ? lo : N);
      lh = (int)(p < N - 1 ? p : N - 1);
    }
    const int r0 = wave_max(lh), r1 = wave_min(lh >= 0 ? rl : 0x7fffffff);
    if (lane == 0) { range[k][0][wave] = r0; range[k][1][wave] = r1; }
  };
  auto collect_range = [&](int k, int& n_tiles, int& full) {
    int rg0 = range[k][0][0], rg1 = range[k][1][0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) { rg0 = max(rg0, range[k][0][w]); rg1 = min(rg1, range[k][1][w]); }
    rg0 = __builtin_amdgcn_readfirstlane(rg0);
    rg1 = __builtin_amdgcn_readfirstlane(rg1);
    n_tiles = rg0 >= 0 ? rg0 / NT + 1 : 0;
    full = rg1 == 0x7fffffff ? 0 : rg1 / NT;
  };

  // The job: row tile qt, key tiles [t0, t1). A split tile runs as pieces
  // of consecutive key tiles whose dQ partials dense_bwd_merge adds. Slot
  // mode (a.q_pair == 0): slot k takes piece k / n_qtiles of row tile
  // n_qtiles-1-k % n_qtiles (tiles longer than q_split run as q_pieces
  // pieces of ceil(n / q_pieces) key tiles; a piece may be empty and then
  // stores zeros). Pair mode (two pieces): row
  // tiles L = n-1-j and S = j form pair j; slot j takes L whole or its first
  // piece, slot P+j takes S whole, slot 2P+odd+j L's second piece if L is
  // split (only where that beats L whole, counting kQPieceCost tiles for the
  // extra piece), an odd middle tile runs whole.
  int qt, piece = 0, n_tiles, full, t0 = 0, t1;
  int64_t pmine;  // this lane's row position in row tile qt (-1: none)
  bool split = false;
  const int P = n_qtiles / 2, odd = n_qtiles & 1;
  const bool middle = a.q_pair && odd && slot == 2 * P;
  if (a.q_pair && !middle) {
    const int j = slot < P ? slot : (slot < 2 * P ? slot - P : slot - 2 * P - odd);
    const int L = n_qtiles - 1 - j;
    int nL, fL, nS, fS;
    // both row tiles' positions in flight together, one barrier
    const int64_t pL = row_pos(L), pS = row_pos(j);
    publish_range(pL, 0);
    publish_range(pS, 1);
    __syncthreads();
    collect_range(0, nL, fL);
    collect_range(1, nS, fS);
    const int h = min(nL, (nL + nS + kQPieceCost + 1) / 2);
    const bool sp = h > 0 && h < nL && max(h, nL - h + nS + kQPieceCost) < nL;
    if (slot < P) {
      qt = L;
      split = sp;
      t1 = sp ? h : nL;
    } else if (slot < 2 * P) {
      qt = j;
      t1 = nS;
    } else {
      if (!sp) return;  // whole workgroup: L ran whole
      qt = L;
      split = true;
      piece = 1;
      t0 = h;
      t1 = nL;
    }
    n_tiles = qt == L ? nL : nS;
    full = qt == L ? fL : fS;
    pmine = qt == L ? pL : pS;
  } else {
    piece = middle ? 0 : slot / n_qtiles;
    qt = middle ? P : n_qtiles - 1 - slot % n_qtiles;
    pmine = row_pos(qt);
    publish_range(pmine, 0);
    __syncthreads();
    collect_range(0, n_tiles, full);
    split = !middle && n_tiles > a.q_split;
    const int h = (n_tiles + a.q_pieces - 1) / a.q_pieces;  // tiles per piece
    t0 = split ? min(piece * h, n_tiles) : 0;
    t1 = split ? min(t0 + h, n_tiles) : n_tiles;
    if (piece && !split) return;  // whole workgroup
  }
  const int row = qt * 32 * WAVES + wave * 32 + col;
  const bool row_in = row < a.Q;
  const int64_t p = pmine;

  // remote keys [0, rlim), local keys [rlim, lhi]; bases of the exponents
  // (+inf for rows without any key, so that every u of theirs is 0)
  int rlim = 0, lhi = -1;
  float base_r = kInf, base_l = kInf, ezrz = 0.f, dl = 0.f, rho = 0.f;
  if (p >= 0) {
    const int64_t c = p >> LOGB;
    const int64_t lo = (c - 1) * b > 0 ? (c - 1) * b : 0;
    rlim = (int)(lo < N ? lo : N);
    lhi = (int)(p < N - 1 ? p : N - 1);
    const int64_t sidx = ((int64_t)bi * a.Q + row) * H + hh;
    const float zr = a.zr[sidx], z = a.z[sidx];
    base_l = z * kLog2e;
    if (zr != kNegInf) {
      base_r = zr * kLog2e;
      ezrz = __expf(zr - z);
    }
  }
  (void)n_tiles;
  // The item's first piece: whether the item was split (for the merge), and
  // per row the last visible key (min(p, N-1); -1 for padding rows and rows
  // beyond Q), per 64-row tile its min and max (for the dK/dV kernel).
  if (piece == 0) {
    const int64_t item = (int64_t)bh * n_qtiles + qt;
    if (threadIdx.x == 0) a.q_count[item] = split ? 1 : 0;
    if (hh == 0) {
      const int lim = p >= 0 ? (int)(p < N - 1 ? p : N - 1) : -1;
      if (row < a.Qp && half == 0) a.lim[(int64_t)bi * a.Qp + row] = lim;
      const int mx = wave_max(lim), mn = wave_min(lim);
      if (lane == 0) { lim_mm[0][wave] = mn; lim_mm[1][wave] = mx; }
      __syncthreads();
      const int rt = row / kRT;  // the 64-row tile of waves 2w' and 2w'+1
      if (lane == 0 && (wave & 1) == 0 && rt < a.Qp / kRT) {
        a.tmin[(int64_t)bi * (a.Qp / kRT) + rt] = min(lim_mm[0][wave], lim_mm[0][wave + 1]);
        a.tmax[(int64_t)bi * (a.Qp / kRT) + rt] = max(lim_mm[1][wave], lim_mm[1][wave + 1]);
      }
    }
  }

  const T* kg = reinterpret_cast<const T*>(a.k) + ((int64_t)bi * N * H + hh) * D;
  const T* vg = reinterpret_cast<const T*>(a.v) + ((int64_t)bi * N * H + hh) * D;
  const int64_t kstride = H * D;
  const Stager<T, DP, WAVES> kst(kg, kstride, a.N), vst(vg, kstride, a.N);
  auto stage = [&]<int BUF>(int i) {
    kst.template stage<NT>(BUF ? k1s : k0s, i * NT);
    vst.template stage<NT>(BUF ? v1s : v0s, i * NT);
  };
  if (t1 > t0) stage.template operator()<0>(t0);

  const int64_t obase = (((int64_t)bi * a.Q + (row_in ? row : 0)) * H + hh) * D;
  Frag qf[NKC], gf[NKC];
  {
    const T* qrow = reinterpret_cast<const T*>(a.q) + obase;
    const T* grow = reinterpret_cast<const T*>(a.dout) + obase;
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      qf[c] = row_in ? *reinterpret_cast<const Frag*>(qrow + c * 16 + half * 8) : Frag{};
      gf[c] = row_in ? *reinterpret_cast<const Frag*>(grow + c * 16 + half * 8) : Frag{};
    }
  }
  // delta = dO.O and rho = dO.RC - delta*PR of this lane's row
  // (st/ops/kernels/dense.py:89-100): this lane's half of the head dim, then
  // the other half's from lane ^ 32
  {
    const T* orow = reinterpret_cast<const T*>(a.out) + obase;
    const float* rrow = a.rc + obase;
    float dsum = 0.f, rsum = 0.f;
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      const Frag o = *reinterpret_cast<const Frag*>(orow + c * 16 + half * 8);
      const f32x4 r0 = *reinterpret_cast<const f32x4*>(rrow + c * 16 + half * 8);
      const f32x4 r1 = *reinterpret_cast<const f32x4*>(rrow + c * 16 + half * 8 + 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float g = to_float<T>(gf[c][e]);
        dsum = fmaf(g, to_float<T>(o[e]), dsum);
        rsum = fmaf(g, e < 4 ? r0[e] : r1[e - 4], rsum);
      }
    }
    dsum += __shfl_xor(dsum, 32, 64);
    rsum += __shfl_xor(rsum, 32, 64);
    if (p >= 0) {
      dl = dsum;
      rho = rsum - dsum * a.pr[((int64_t)bi * a.Q + row) * H + hh];
    }
  }

  // per-lane LDS fragment offsets (see dense_fwd_fast.hip)
  int koff[NKC];
#pragma unroll
  for (int c = 0; c < NKC; ++c) koff[c] = col * DP + (((2 * c + half) ^ swz<DP>(col)) * 8);
  int toff[NDT], toff8[NDT];  // rows r0 and r0 + 8 (swizzled separately)
  {
    const int gi = lane >> 4, sl = lane & 15;
    const int r0 = 4 * (gi >> 1) + (sl >> 2);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d = 32 * dt + 16 * (gi & 1) + 4 * (sl & 3);
      toff[dt] = r0 * DP + (((d >> 3) ^ swz<DP>(r0)) * 8) + (d & 7);
      toff8[dt] = (r0 + 8) * DP + (((d >> 3) ^ swz<DP>(r0 + 8)) * 8) + (d & 7);
    }
  }
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef short s8 __attribute__((ext_vector_type(8)));
  auto rfrag = [&](const T* buf, int st, int c) -> Frag {
    return *reinterpret_cast<const Frag*>(buf + 32 * st * DP + koff[c]);
  };
  auto tfrag = [&](const T* buf, int k0, int dt) -> Frag {
    const T* p0 = buf + k0 * DP + toff[dt];
    const T* p1 = buf + k0 * DP + toff8[dt];
    s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)p0);
    s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)p1);
    return __builtin_bit_cast(Frag, (s8)__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  f32x16 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc[dt] = zero16();
  constexpr bool AUG = AugTable<T, LOGB>::on;
  float2* tab = a.tab + (int64_t)bh * a.nblk * a.Qp;
  bf16x8* taug = reinterpret_cast<bf16x8*>(a.tab) + (int64_t)bh * a.nblk * a.Qp;
  const float inv_c2 = 1.f / a.scale_log2;
  const float c2 = a.scale_log2;

  auto step = [&]<int BUF, bool FULL>(int i) {
    const int kb = i * NT;
    wait_vm();
    __syncthreads();
    if (i + 1 < t1) stage.template operator()<1 - BUF>(i + 1);
    const T* kt = BUF ? k1s : k0s;
    const T* vt = BUF ? v1s : v0s;

    f32x16 s[NST], dp[NST];
#pragma unroll
    for (int st = 0; st < NST; ++st) { s[st] = zero16(); dp[st] = zero16(); }
    // key of register r in subtile st: kb + 4*half + off(st, r)
    const int base_k = kb + 4 * half;
    const int lim_v = lhi + 1 - base_k;  // visible iff off < lim_v
    auto offset = [](int st, int r) { return 32 * st + 8 * (r >> 2) + (r & 3); };
    // Remote-ness is constant over a key block (the remote limit is block
    // aligned), so it is one flag per block slot; only visibility (the
    // causal limit) varies per key. Per slot: the exponent base, the
    // multiplier P/u (U_j e^{ZR-Z} remote, 1 local) and the gate coefficient.
    constexpr int NS = BlkSlots<LOGB>::n;
    bool remb[NST][NS];
    float nbase[NST][NS];
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        remb[st][j] = FULL || (blk_index<LOGB>(st, j, half) << LOGB) < rlim - kb;
        nbase[st][j] = remb[st][j] ? -base_r : -base_l;
      }
    // u of subtile ST, registers 8H..8H+7
    auto expo = [&]<int ST, int H>() {
#pragma unroll
      for (int r = 8 * H; r < 8 * H + 8; ++r) {
        const float x = fmaf(s[ST][r], c2, nbase[ST][blk_slot<LOGB>(r)]);
        if constexpr (FULL) s[ST][r] = fast_exp2(x);
        else s[ST][r] = offset(ST, r) < lim_v ? fast_exp2(x) : 0.f;
      }
    };
    // in-lane parts of U_j (sums of u) and X_j (sums of u dP) of subtile ST
    float up[NST][8], xp[NST][8];
    auto part = [&]<int ST>() {
      block_part<LOGB, false>(s[ST], s[ST], up[ST]);
      block_part<LOGB, true>(s[ST], dp[ST], xp[ST]);
    };
    // The tile's finish, once the last subtile's in-lane sums are in: U_j
    // and X_j = sum u_i dP_i per block, the multipliers, the gate
    // coefficients and the table entries. With m_j = P_i / u_i (U_j
    // e^{ZR-Z} remote, 1 local), G_j = m_j (X_j - delta U_j), so the gate
    // coefficient G_j / U_j - rho is e^{ZR-Z} (X_j - delta U_j) - rho on
    // remote blocks (0 where U_j = 0: every u is 0) and 0 on local ones, and
    //   dA_i = P_i (dP_i - delta) + u_i gb_j = u_i (m_j dP_i + c_j),
    //   c_j = gb_j - m_j delta.
    float mult[NST][NS], cb[NST][NS];
    Frag bd[NST][2];
    auto finish = [&]() {
      float ub[NST][8], xb[NST][8], gb[NST][8];
      block_finish<NST, LOGB>(up, ub);
      block_finish<NST, LOGB>(xp, xb);
#pragma unroll
      for (int st = 0; st < NST; ++st)
#pragma unroll
        for (int j = 0; j < NS; ++j) {
          mult[st][j] = remb[st][j] ? ub[st][j] * ezrz : 1.f;
          gb[st][j] = remb[st][j] && ub[st][j] > 0.f ? ezrz * fmaf(-dl, ub[st][j], xb[st][j]) - rho : 0.f;
          cb[st][j] = fmaf(-mult[st][j], dl, gb[st][j]);
        }
      // table entries of this tile's blocks (one writer per row and block)
      if (row_in && (BlkSlots<LOGB>::per_half || half == 0)) {
        constexpr int STEP = LOGB >= 5 ? ((1 << LOGB) / 32 < NST ? (1 << LOGB) / 32 : NST) : 1;
#pragma unroll
        for (int st = 0; st < NST; st += STEP)
#pragma unroll
          for (int j = 0; j < NS; ++j) {
            const int bl = (kb >> LOGB) + blk_index<LOGB>(st, j, half);
            const int ks = bl << LOGB;
            float beta, eps;
            if (FULL || ks < rlim) {
              const float u = ub[st][j];
              beta = base_l - fast_log2(u);
              const float w = u * ezrz;
              float gam = w > 0.f ? gb[st][j] / w : 0.f;
              gam = fabsf(gam) <= 3.0e38f ? gam : 0.f;  // overflow only where P_i is 0
              eps = gam - dl;
            } else if (ks <= lhi) {
              beta = base_l;
              eps = -dl;
            } else {
              beta = kInf;
              eps = 0.f;
            }
            if constexpr (AUG) {
              // the terms of -beta/c2 (+inf: a large finite value), then of eps
              bf16 tb_[3], te_[3];
              split3_bf16(fmaxf(fminf(-beta * inv_c2, 1e30f), -1e30f), tb_);
              split3_bf16(eps, te_);
              const bf16 z = (bf16)0.f;
              taug[(int64_t)bl * a.Qp + row] = bf16x8{tb_[0], tb_[1], tb_[2], te_[0], te_[1], te_[2], z, z};
            } else {
              tab[(int64_t)bl * a.Qp + row] = make_float2(beta, eps);
            }
          }
      }
    };
    // dA of subtile ST (direct + gate term) as 16-bit MFMA operands
    auto gate = [&]<int ST>() {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        dp[ST][r] = s[ST][r] * fmaf(mult[ST][blk_slot<LOGB>(r)], dp[ST][r], cb[ST][blk_slot<LOGB>(r)]);
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) bd[ST][h2] = frag_from_c<T>(dp[ST], h2);
    };
    // One chain of products per tile, one chunk (4 MFMAs) of LDS reads
    // ahead throughout: S^T = K Q^T and dP^T = V dO^T of each subtile (2 NKC
    // products, S even, dP odd), then dQ^T += K^T dA^T (2 NDT products per
    // subtile: 16-key chunk 2ST + k/NDT, head-dim tile k % NDT). Beside the
    // S/dP products of subtile ST run the exponentials and in-lane sums of
    // subtile ST-1; after the last ones, the tile's finish and the first
    // gate (the reads of the first dQ chunk already in flight); beside the
    // dQ products of subtile ST, the gate of subtile ST+1.
    constexpr int P1 = 2 * NKC, P2 = 2 * NDT, N1 = NST * P1;
    constexpr int CP1 = P1 / 4, CP2 = P2 / 4, C1 = NST * CP1, C2 = NST * CP2;
    static_assert(P1 % 4 == 0 && P2 % 4 == 0, "whole chunks per subtile");
    auto load = [&]<int J>() -> Frag {
      if constexpr (J < N1) {
        constexpr int st = J / P1, jj = J % P1;
        return rfrag((jj & 1) ? vt : kt, st, jj >> 1);
      } else {
        constexpr int jj = J - N1, st = jj / P2, k = jj % P2;
        return tfrag(kt, 16 * (2 * st + k / NDT), k % NDT);
      }
    };
    auto mma = [&]<int J>(Frag f) {
      if constexpr (J < N1) {
        constexpr int st = J / P1, jj = J % P1;
        if constexpr (jj & 1) dp[st] = M::mma(f, gf[jj >> 1], dp[st]);
        else s[st] = M::mma(f, qf[jj >> 1], s[st]);
      } else {
        constexpr int jj = J - N1, st = jj / P2, k = jj % P2;
        acc[k % NDT] = M::mma(f, bd[st][k / NDT], acc[k % NDT]);
      }
    };
    auto after = [&]<int G>() {
      if constexpr (G < C1) {
        constexpr int st = G / CP1, lg = G % CP1;
        if constexpr (st >= 1) {
          // slices [lg*3/CP1, (lg+1)*3/CP1) of subtile st-1: the two halves
          // of its exponentials, then its in-lane sums
          [&]<int... K>(std::integer_sequence<int, K...>) {
            ([&] {
              constexpr int k = lg * 3 / CP1 + K;
              if constexpr (k < 2) expo.template operator()<st - 1, k>();
              else part.template operator()<st - 1>();
            }(), ...);
          }(std::make_integer_sequence<int, (lg + 1) * 3 / CP1 - lg * 3 / CP1>{});
        }
        if constexpr (G == C1 - 1) {
          expo.template operator()<NST - 1, 0>();
          expo.template operator()<NST - 1, 1>();
          part.template operator()<NST - 1>();
          finish();
          gate.template operator()<0>();
        }
      } else {
        constexpr int st = (G - C1) / CP2, lg = (G - C1) % CP2;
        if constexpr (lg == CP2 - 1 && st + 1 < NST) gate.template operator()<st + 1>();
      }
    };
    mfma_chain<C1 + C2, 4>(load, mma, after);
  };
  auto run = [&]<int BUF>(int i) {
    if (i < full) step.template operator()<BUF, true>(i);
    else step.template operator()<BUF, false>(i);
  };
  for (int i = t0; i < t1; i += 2) {
    run.template operator()<0>(i);
    if (i + 1 < t1) run.template operator()<1>(i + 1);
  }
  if (split) {
    const int item = bh * n_qtiles + qt;
    store_piece<NDT>(acc, a.q_part + (size_t)item * a.q_pieces * 4 * (NDT * 16 * 64), piece);
    return;
  }
  if (!row_in) return;
  T* dq = reinterpret_cast<T*>(a.dq) + obase;
  typedef T T4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      T4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = from_float<T>(acc[dt][4 * i + j] * a.scale);
      *reinterpret_cast<T4*>(dq + 32 * dt + 8 * i + 4 * half) = o;
    }
}

// ---------------------------------------------------------------------------
// dK and dV. A workgroup owns 128 keys of one (batch, head) (wave w: keys
// 32w..32w+31, lane = key) and walks the 64-row query tiles that see any of
// them. Score tiles are S = Q K^T and dP = dO V^T (lane = key), K and V
// fragments stay in registers; dV^T += dO^T P and dK^T += Q^T dA take the
// transposed operands from the staged tiles.
template <typename T, int DP, int LOGB>
// (head_dim 64: two workgroups per compute unit, so that one's prologue,
// staging waits and epilogue overlap the other's products; at 128 the
// registers allow one)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DP == 64 ? 2 : 1, DP == 64 ? 2 : 1))) void dense_bwd_dkv_fast_kernel(DenseArgs a, int n_rtiles, int n_ktiles) {
  typedef Mma<T> M;
  typedef typename M::Frag Frag;
  constexpr int WAVES = 4;
  constexpr int MQ = kRT;
  constexpr int NRS = MQ / 32;
  constexpr int NDT = DP / 32;
  constexpr int NKC = DP / M::KW;
  constexpr int QTILE = MQ * DP;
  constexpr int NB = (kKT >> LOGB) > 0 ? (kKT >> LOGB) : 1;  // key blocks per workgroup
  __shared__ __attribute__((aligned(16))) T q0s[QTILE];
  __shared__ __attribute__((aligned(16))) T q1s[QTILE];
  __shared__ __attribute__((aligned(16))) T g0s[QTILE];
  __shared__ __attribute__((aligned(16))) T g1s[QTILE];
  constexpr bool AUG = AugTable<T, LOGB>::on;
  constexpr int TENT = AugTable<T, LOGB>::bytes;
  __shared__ __attribute__((aligned(16))) char t0s[NB * MQ * TENT];
  __shared__ __attribute__((aligned(16))) char t1s[NB * MQ * TENT];
  __shared__ __attribute__((aligned(16))) int l0s[MQ];
  __shared__ __attribute__((aligned(16))) int l1s[MQ];
  __shared__ int list[kMaxRTiles];
  __shared__ int count;

  __shared__ int pair_rows[2];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int BH = a.B * a.H;
  const int bh = blockIdx.x % BH, slot = (int)(blockIdx.x / BH);
  const int bi = bh / a.H, hh = bh % a.H;
  const int64_t H = a.H, D = a.D, N = a.N;
  const int64_t kstride = H * D;
  const int* tmax = a.tmax + (int64_t)bi * n_rtiles;
  const int* tmin = a.tmin + (int64_t)bi * n_rtiles;

  // The job: key tile kt_idx, active row tiles [i0, i1) of its list. A
  // split tile runs as two pieces whose dK/dV partials dense_bwd_merge adds.
  // Slot mode (a.k_pair == 0): slot k < n_ktiles takes key tile k whole or
  // its first half, slot n_ktiles+k its second half (tiles seen by more
  // than k_split row tiles are halved; ascending key tiles, the first see
  // the most rows). Pair mode: key tiles L = j and S = n-1-j form pair j;
  // slot j takes L whole or its first piece, slot P+j takes S whole, slot
  // 2P+odd+j L's second piece if L is split (only where that beats L whole,
  // counting kKPieceCost row tiles for the extra piece); an odd middle tile
  // runs whole.
  int kt_idx, piece = 0, hsplit = 0;
  bool split = false;
  const int P = n_ktiles / 2, odd = n_ktiles & 1;
  const bool middle = a.k_pair && odd && slot == 2 * P;
  int pj = 0;
  if (a.k_pair && !middle) {
    pj = slot < P ? slot : (slot < 2 * P ? slot - P : slot - 2 * P - odd);
    if (wave == 0) {
      // row tiles reaching key tiles L and S
#pragma unroll
      for (int which = 0; which < 2; ++which) {
        const int kb_w = (which ? n_ktiles - 1 - pj : pj) * kKT;
        int n = 0;
        for (int c0 = 0; c0 < n_rtiles; c0 += 64) {
          const int t = c0 + lane;
          n += __popcll(__ballot(t < n_rtiles && tmax[t] >= kb_w));
        }
        if (lane == 0) pair_rows[which] = n;
      }
    }
    __syncthreads();
    const int nL = pair_rows[0], nS = pair_rows[1];
    const int h = min(nL, (nL + nS + kKPieceCost + 1) / 2);
    const bool sp = h > 0 && h < nL && max(h, nL - h + nS + kKPieceCost) < nL;
    if (slot < P) {
      kt_idx = pj;
      split = sp;
    } else if (slot < 2 * P) {
      kt_idx = n_ktiles - 1 - pj;
    } else {
      if (!sp) return;  // whole workgroup: L ran whole
      kt_idx = pj;
      split = true;
      piece = 1;
    }
    hsplit = h;
  } else {
    piece = !middle && slot >= n_ktiles;
    kt_idx = middle ? P : (piece ? slot - n_ktiles : slot);
  }
  const int kb = kt_idx * kKT;
  const int key = kb + 32 * wave + col;

  // No row reaches these keys (every row tile's last visible key is below
  // kb): dK = dV = 0. Each wave decides by itself (one load per lane and
  // 64 row tiles) and writes its 32 zero rows with 16-byte stores, before
  // any K/V load.
  {
    bool any = false;
    for (int c0 = 0; c0 < n_rtiles && !any; c0 += 64) {
      const int t = c0 + lane;
      any = __ballot(t < n_rtiles && tmax[t] >= kb) != 0;
    }
    if (!any) {
      if (piece) return;  // the tile's first slot writes the zeros
      if (threadIdx.x == 0) a.k_count[(int64_t)bh * n_ktiles + kt_idx] = 0;
      constexpr int LPR = DP * (int)sizeof(T) / 16;  // lanes per key row
      constexpr int RPI = 64 / LPR;                   // rows per store instruction
      typedef typename Vec16<T>::type V;
#pragma unroll
      for (int it = 0; it < 32 / RPI; ++it) {
        const int k = kb + 32 * wave + it * RPI + lane / LPR;
        if (k < a.N) {
          const int64_t off = (((int64_t)bi * N + k) * H + hh) * D + (lane % LPR) * Vec16<T>::n;
          *reinterpret_cast<V*>(reinterpret_cast<T*>(a.dk) + off) = V{};
          *reinterpret_cast<V*>(reinterpret_cast<T*>(a.dv) + off) = V{};
        }
      }
      return;
    }
  }

  // row tiles that see a key of this workgroup, in order; bit 0 marks tiles
  // whose rows all see every key of it (no masks)
  if (wave == 0) {
    int n = 0;
    for (int c0 = 0; c0 < n_rtiles; c0 += 64) {
      const int t = c0 + lane;
      const int mx = t < n_rtiles ? tmax[t] : -1;
      const int mn = t < n_rtiles ? tmin[t] : -1;
      const bool act = mx >= kb;
      const uint64_t m = __ballot(act);
      const int before = __popcll(m & ((uint64_t(1) << lane) - 1));
      if (act) list[n + before] = 2 * t + (mn >= kb + kKT - 1 ? 1 : 0);
      n += __popcll(m);
    }
    if (lane == 0) count = n;
  }

  const T* kg = reinterpret_cast<const T*>(a.k) + ((int64_t)bi * N * H + hh) * D;
  const T* vg = reinterpret_cast<const T*>(a.v) + ((int64_t)bi * N * H + hh) * D;
  Frag kf[NKC], vf[NKC];
  {
    const bool key_in = key < a.N;
    const T* krow = kg + (int64_t)(key_in ? key : 0) * kstride;
    const T* vrow = vg + (int64_t)(key_in ? key : 0) * kstride;
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      kf[c] = key_in ? *reinterpret_cast<const Frag*>(krow + c * 16 + half * 8) : Frag{};
      vf[c] = key_in ? *reinterpret_cast<const Frag*>(vrow + c * 16 + half * 8) : Frag{};
    }
  }
  __syncthreads();
  const int n_act = count;
  if (!a.k_pair || middle) {
    split = !middle && n_act > a.k_split;
    hsplit = (n_act + 1) / 2;
    if (piece && !split) return;  // whole workgroup
  }
  if (piece == 0 && threadIdx.x == 0) a.k_count[(int64_t)bh * n_ktiles + kt_idx] = split ? 1 : 0;
  const int i0 = split && piece ? hsplit : 0;
  const int i1 = split && !piece ? hsplit : n_act;

  const T* qg = reinterpret_cast<const T*>(a.q) + ((int64_t)bi * a.Q * H + hh) * D;
  const T* gg = reinterpret_cast<const T*>(a.dout) + ((int64_t)bi * a.Q * H + hh) * D;
  const char* tg = reinterpret_cast<const char*>(a.tab) + ((int64_t)bh * a.nblk + (int64_t)kt_idx * NB) * a.Qp * TENT;
  const int* lg = a.lim + (int64_t)bi * a.Qp;
  const Stager<T, DP, WAVES> qst(qg, kstride, a.Q), gst(gg, kstride, a.Q);
  auto stage = [&]<int BUF>(int idx) {
    const int m0 = (list[idx] >> 1) * MQ;
    qst.template stage<MQ>(BUF ? q1s : q0s, m0);
    gst.template stage<MQ>(BUF ? g1s : g0s, m0);
    // table slice: NB blocks x 64 rows, 64 * TENT contiguous bytes per
    // block, 16 bytes per lane (two float2 rows, or one entry)
    char* tl = BUF ? t1s : t0s;
    constexpr int CPB = MQ * TENT / 16;  // copies per block
#pragma unroll
    for (int j0 = 0; j0 < NB * CPB; j0 += 256) {
      const int j = j0 + (int)threadIdx.x;
      if (j < NB * CPB)
        async_copy16(tg + ((int64_t)(j / CPB) * a.Qp + m0) * TENT + (j % CPB) * 16, tl + (j0 + 64 * wave) * 16);
    }
    if (threadIdx.x < 16) async_copy16(lg + m0 + 4 * threadIdx.x, BUF ? l1s : l0s);
  };
  if (i1 > i0) stage.template operator()<0>(i0);

  int qoff[NKC];
#pragma unroll
  for (int c = 0; c < NKC; ++c) qoff[c] = col * DP + (((2 * c + half) ^ swz<DP>(col)) * 8);
  int toff[NDT], toff8[NDT];  // rows r0 and r0 + 8 (swizzled separately)
  {
    const int gi = lane >> 4, sl = lane & 15;
    const int r0 = 4 * (gi >> 1) + (sl >> 2);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d = 32 * dt + 16 * (gi & 1) + 4 * (sl & 3);
      toff[dt] = r0 * DP + (((d >> 3) ^ swz<DP>(r0)) * 8) + (d & 7);
      toff8[dt] = (r0 + 8) * DP + (((d >> 3) ^ swz<DP>(r0 + 8)) * 8) + (d & 7);
    }
  }
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef short s8 __attribute__((ext_vector_type(8)));
  auto rfrag = [&](const T* buf, int rs, int c) -> Frag {
    return *reinterpret_cast<const Frag*>(buf + 32 * rs * DP + qoff[c]);
  };
  auto tfrag = [&](const T* buf, int k0, int dt) -> Frag {
    const T* p0 = buf + k0 * DP + toff[dt];
    const T* p1 = buf + k0 * DP + toff8[dt];
    s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)p0);
    s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)p1);
    return __builtin_bit_cast(Frag, (s8)__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  f32x16 dk[NDT], dv[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) { dk[dt] = zero16(); dv[dt] = zero16(); }
  const int tcol = ((32 * wave + col) >> LOGB) * MQ * TENT;  // this lane's block in the table slice (bytes)
  const float c2 = a.scale_log2;
  // AugTable: B operands of the table's contraction chunk (k = 0..7 the
  // entry, 8..15 zero rows): ones against the terms of -beta/c2 (k = 0..2)
  // for S and of eps (k = 3..5) for dP
  Frag ones_s = {}, ones_dp = {};
  if constexpr (AUG) {
    const T o = (T)1.f, z = (T)0.f;
    ones_s = half ? Frag{} : Frag{o, o, o, z, z, z, z, z};
    ones_dp = half ? Frag{} : Frag{z, z, z, o, o, o, z, z};
  }

  auto step = [&]<int BUF, bool FULL>(int idx) {
    wait_vm();
    __syncthreads();
    if (idx + 1 < i1) stage.template operator()<1 - BUF>(idx + 1);
    const T* qt = BUF ? q1s : q0s;
    const T* gt = BUF ? g1s : g0s;
    const char* tb = (BUF ? t1s : t0s) + tcol;
    const float* tt = reinterpret_cast<const float*>(tb);
    const int* lt = BUF ? l1s : l0s;

    // AugTable: the table's chunk starts S (-beta/c2) and dP (eps)
    f32x16 s[NRS], dp[NRS];
    if constexpr (!AUG) {
#pragma unroll
      for (int rs = 0; rs < NRS; ++rs) { s[rs] = zero16(); dp[rs] = zero16(); }
    }
    Frag bp[NRS][2], bd[NRS][2];
    // Elementwise work of row subtile RS, slice I: register group I (rows
    // 32RS + 8I + 4half + 0..3) for I < 4, then the conversion of P and dA
    // to 16-bit MFMA operands (row order permuted as in frag_from_c).
    auto elem = [&]<int RS, int I>() {
      if constexpr (I < 4) {
        const int r0 = 32 * RS + 8 * I + 4 * half;
        float beta[4] = {0.f, 0.f, 0.f, 0.f}, eps[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (!AUG) {
          const f32x4 t01 = *reinterpret_cast<const f32x4*>(tt + 2 * r0);
          const f32x4 t23 = *reinterpret_cast<const f32x4*>(tt + 2 * r0 + 4);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            beta[j] = t01[2 * j];
            eps[j] = t01[2 * j + 1];
            beta[2 + j] = t23[2 * j];
            eps[2 + j] = t23[2 * j + 1];
          }
        }
        int lim[4] = {0, 0, 0, 0};
        if constexpr (!FULL) {
          typedef int i4 __attribute__((ext_vector_type(4)));
          const i4 l4 = *reinterpret_cast<const i4*>(lt + r0);
#pragma unroll
          for (int j = 0; j < 4; ++j) lim[j] = l4[j];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * I + j;
          // AugTable: S and dP already hold -beta/c2 and eps
          const float pv = AUG ? fast_exp2(s[RS][r] * c2) : fast_exp2(fmaf(s[RS][r], c2, -beta[j]));
          const float da = AUG ? pv * dp[RS][r] : pv * (dp[RS][r] + eps[j]);
          if constexpr (FULL) {
            s[RS][r] = pv;
            dp[RS][r] = da;
          } else {
            const bool vis = key <= lim[j];
            s[RS][r] = vis ? pv : 0.f;
            dp[RS][r] = vis ? da : 0.f;
          }
        }
      } else {
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          bp[RS][h2] = frag_from_c<T>(s[RS], h2);
          bd[RS][h2] = frag_from_c<T>(dp[RS], h2);
        }
      }
    };
    // One chain of products per step, one chunk (4 MFMAs) of LDS reads
    // ahead throughout: S = Q K^T and dP = dO V^T of row subtile 0, then of
    // subtile 1 (2 NKC products each: chunk j/2, S even, dP odd), then
    // dV^T += dO^T P and dK^T += Q^T dA over the rows of subtile 0, then of
    // subtile 1 (4 NDT products each: 16-row chunk 2RS + j/(2NDT), head-dim
    // tile (j/2) % NDT, dV even, dK odd). Subtile 0's elementwise work runs
    // beside subtile 1's S/dP products, subtile 1's beside subtile 0's
    // dK/dV products.
    static_assert(NRS == 2, "two row subtiles per step");
    // AugTable: a first chunk of four products starts S and dP of both row
    // subtiles with the table's terms (row 32RS + col of the lane's block)
    constexpr int NI = AUG ? 4 : 0, CI = NI / 4;
    constexpr int PA = 2 * NKC, PB = 4 * NDT, CA = PA / 4, CB = PB / 4;
    static_assert(PA % 4 == 0 && PB % 4 == 0, "whole chunks per subtile");
    auto load = [&]<int J0>() -> Frag {
      constexpr int J = J0 - NI;
      if constexpr (J < 0) {
        return *reinterpret_cast<const Frag*>(tb + (32 * ((J0 >> 1) & 1) + col) * TENT);
      } else if constexpr (J < 2 * PA) {
        constexpr int rs = J / PA, j = J % PA;
        return rfrag((j & 1) ? gt : qt, rs, j >> 1);
      } else {
        constexpr int rs = (J - 2 * PA) / PB, j = (J - 2 * PA) % PB;
        return tfrag((j & 1) ? qt : gt, 16 * (2 * rs + j / (2 * NDT)), (j >> 1) % NDT);
      }
    };
    auto mma = [&]<int J0>(Frag f) {
      constexpr int J = J0 - NI;
      if constexpr (J < 0) {
        constexpr int rs = (J0 >> 1) & 1;
        if constexpr (J0 & 1) dp[rs] = M::mma(f, ones_dp, zero16());
        else s[rs] = M::mma(f, ones_s, zero16());
      } else if constexpr (J < 2 * PA) {
        constexpr int rs = J / PA, j = J % PA;
        if constexpr (j & 1) dp[rs] = M::mma(f, vf[j >> 1], dp[rs]);
        else s[rs] = M::mma(f, kf[j >> 1], s[rs]);
      } else {
        constexpr int rs = (J - 2 * PA) / PB, j = (J - 2 * PA) % PB;
        constexpr int h2 = j / (2 * NDT), dt = (j >> 1) % NDT;
        if constexpr (j & 1) dk[dt] = M::mma(f, bd[rs][h2], dk[dt]);
        else dv[dt] = M::mma(f, bp[rs][h2], dv[dt]);
      }
    };
    // slices [lg*5/C, (lg+1)*5/C) of a subtile's elementwise work after
    // chunk lg of the C chunks it runs beside
    auto slices = [&]<int RS, int LG, int C>() {
      [&]<int... K>(std::integer_sequence<int, K...>) {
        (elem.template operator()<RS, LG * 5 / C + K>(), ...);
      }(std::make_integer_sequence<int, (LG + 1) * 5 / C - LG * 5 / C>{});
    };
    auto after = [&]<int G0>() {
      constexpr int G = G0 - CI;
      if constexpr (G >= CA && G < 2 * CA) slices.template operator()<0, G - CA, CA>();
      else if constexpr (G >= 2 * CA && G < 2 * CA + CB) slices.template operator()<1, G - 2 * CA, CB>();
    };
    mfma_chain<CI + 2 * CA + 2 * CB, 4>(load, mma, after);
  };
  auto run = [&]<int BUF>(int idx) {
    if (list[idx] & 1) step.template operator()<BUF, true>(idx);
    else step.template operator()<BUF, false>(idx);
  };
  for (int idx = i0; idx < i1; idx += 2) {
    run.template operator()<0>(idx);
    if (idx + 1 < i1) run.template operator()<1>(idx + 1);
  }
  if (split) {
    f32x16 both[2 * NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) { both[dt] = dk[dt]; both[NDT + dt] = dv[dt]; }
    const int item = bh * n_ktiles + kt_idx;
    store_piece<2 * NDT>(both, a.k_part + (size_t)item * 2 * 4 * (2 * NDT * 16 * 64), piece);
    return;
  }
  if (key >= a.N) return;
  const int64_t kbase = (((int64_t)bi * N + key) * H + hh) * D;
  T* dkp = reinterpret_cast<T*>(a.dk) + kbase;
  T* dvp = reinterpret_cast<T*>(a.dv) + kbase;
  typedef T T4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      T4 ok, ov;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ok[j] = from_float<T>(dk[dt][4 * i + j] * a.scale);
        ov[j] = from_float<T>(dv[dt][4 * i + j]);
      }
      *reinterpret_cast<T4*>(dkp + 32 * dt + 8 * i + 4 * half) = ok;
      *reinterpret_cast<T4*>(dvp + 32 * dt + 8 * i + 4 * half) = ov;
    }
}

// ---------------------------------------------------------------------------
// Sum of the pieces of every split item (q_pieces for dQ, two for dK/dV):
// workgroup (w, t) with
// w < n_qitems handles accumulator tile t of dQ item w (128 rows), the rest
// the dK/dV items (128 keys; tiles 0..NDT-1 dK, NDT.. dV). Thread (wave,
// lane) holds the registers of the same (wave, lane) of the piece kernels,
// i.e. row/key 32*wave + lane%32 and dims 32*dt + 8*(r/4) + 4*(lane/32) + r%4.
// Sum over NP pieces of one accumulator tile's 16 registers of this lane
// (every load issued before the additions).
template <int NP>
__device__ __forceinline__ void sum_pieces(const float* p0, size_t pstride, int t, float (&out)[16]) {
  const int lane = threadIdx.x & 63;
  f32x4 v[NP][4];
#pragma unroll
  for (int q = 0; q < NP; ++q)
#pragma unroll
    for (int i = 0; i < 4; ++i) v[q][i] = reinterpret_cast<const f32x4*>(p0 + q * pstride)[(t * 4 + i) * 64 + lane];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    float s = v[0][e >> 2][e & 3];
#pragma unroll
    for (int q = 1; q < NP; ++q) s += v[q][e >> 2][e & 3];
    out[e] = s;
  }
}

template <typename T, int DP>
__global__ __launch_bounds__(256) void dense_bwd_merge_kernel(DenseArgs a, int n_qtiles, int n_ktiles) {
  constexpr int NDT = DP / 32;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int BH = a.B * a.H;
  const int n_qitems = BH * n_qtiles;
  const bool is_q = (int)blockIdx.x < n_qitems;
  const int item = is_q ? (int)blockIdx.x : (int)blockIdx.x - n_qitems;
  if ((is_q ? a.q_count : a.k_count)[item] == 0) return;
  const int n_t = is_q ? n_qtiles : n_ktiles;
  const int bh = item / n_t, tile = item % n_t;
  const int bi = bh / a.H, hh = bh % a.H;
  const int idx = tile * 128 + wave * 32 + col;  // row (dQ) or key (dK/dV)
  const int64_t H = a.H, D = a.D;
  typedef T T4 __attribute__((ext_vector_type(4)));
  const int nacc = is_q ? NDT : 2 * NDT;
  const int np = is_q ? a.q_pieces : 2;
  const float* p0 = (is_q ? a.q_part : a.k_part) + ((size_t)item * np * 4 + wave) * (nacc * 16 * 64);
  const size_t pstride = (size_t)4 * nacc * 16 * 64;
  if (idx >= (is_q ? a.Q : a.N)) return;
  // one accumulator tile per workgroup (blockIdx.y): dQ has NDT, dK/dV 2*NDT
  const int t = blockIdx.y;
  if (t >= nacc) return;
  {
    const int dt = t % NDT;
    const float sc = (t < NDT) ? a.scale : 1.f;  // dQ and dK carry 1/sqrt(D); dV does not
    T* dst;
    if (is_q) dst = reinterpret_cast<T*>(a.dq) + (((int64_t)bi * a.Q + idx) * H + hh) * D;
    else dst = reinterpret_cast<T*>(t < NDT ? a.dk : a.dv) + (((int64_t)bi * a.N + idx) * H + hh) * D;
    float sum[16];
    if (np == 8) sum_pieces<8>(p0, pstride, t, sum);
    else if (np == 4) sum_pieces<4>(p0, pstride, t, sum);
    else sum_pieces<2>(p0, pstride, t, sum);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      T4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = from_float<T>(sum[4 * i + j] * sc);
      *reinterpret_cast<T4*>(dst + 32 * dt + 8 * i + 4 * half) = o;
    }
  }
}

// Compute units of the current device (cached per device).
static int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

template <typename T, int DP>
static hipError_t launch_fast(const DenseArgs& args, hipStream_t stream) {
  DenseArgs a = args;
  const int n_qtiles = (a.Q + 127) / 128;
  const int n_ktiles = (a.N + kKT - 1) / kKT;
  const int n_rtiles = a.Qp / kRT;
  const unsigned BH = (unsigned)(a.B * a.H);
  // pair mode once slot mode's dQ slots outnumber the compute units
  a.q_pair = 2 * (int64_t)n_qtiles * BH > device_cus();
  if (a.q_pair) a.q_pieces = 2;
  const int q_slots = a.q_pair ? 3 * (n_qtiles / 2) + (n_qtiles & 1) : a.q_pieces * n_qtiles;
  // few query rows (at most kFewRTiles 64-row tiles): every visible key
  // tile carries about the same work, so one workgroup per key tile, never
  // split; else pair mode once slot mode's slots outnumber the compute units
  const bool few_rows = n_rtiles <= kFewRTiles;
  if (few_rows) a.k_split = n_rtiles;
  a.k_pair = !few_rows && 2 * (int64_t)n_ktiles * BH > device_cus();
  const int k_slots = a.k_pair ? 3 * (n_ktiles / 2) + (n_ktiles & 1) : (few_rows ? n_ktiles : 2 * n_ktiles);
  // merge workgroups: the dQ items, then the dK/dV items unless none can be
  // split (few rows)
  const unsigned merge_items = (unsigned)((n_qtiles + (few_rows ? 0 : n_ktiles)) * BH);
  auto go = [&]<int LOGB>() {
    note_launch((const void*)&dense_bwd_dq_fast_kernel<T, DP, LOGB>,
                {"dense_bwd_dq_fast", dtype_code<T>(), DP, 1 << LOGB, 128, 128, 4, 2, q_slots * BH,
                 a.q_pair ? "pair" : "slot"});
    note_launch((const void*)&dense_bwd_dkv_fast_kernel<T, DP, LOGB>,
                {"dense_bwd_dkv_fast", dtype_code<T>(), DP, 1 << LOGB, 128, 64, 4, 2, k_slots * BH,
                 a.k_pair ? "pair" : "slot"});
    note_launch((const void*)&dense_bwd_merge_kernel<T, DP>,
                {"dense_bwd_merge", dtype_code<T>(), DP, 1 << LOGB, 128, DP, 4, 0,
                 merge_items * 2 * (DP / 32), "rows"});
    hipLaunchKernelGGL((dense_bwd_dq_fast_kernel<T, DP, LOGB>), dim3(q_slots * BH), dim3(256), 0, stream,
                       a, n_qtiles);
    if (hipPeekAtLastError() != hipSuccess) return;
    hipLaunchKernelGGL((dense_bwd_dkv_fast_kernel<T, DP, LOGB>), dim3(k_slots * BH), dim3(256), 0,
                       stream, a, n_rtiles, n_ktiles);
    if (hipPeekAtLastError() != hipSuccess) return;
    hipLaunchKernelGGL((dense_bwd_merge_kernel<T, DP>), dim3(merge_items, 2 * (DP / 32)),
                       dim3(256), 0, stream, a, n_qtiles, n_ktiles);
  };
  switch (a.logb) {
    case 1: go.template operator()<1>(); break;
    case 2: go.template operator()<2>(); break;
    case 3: go.template operator()<3>(); break;
    case 4: go.template operator()<4>(); break;
    case 5: go.template operator()<5>(); break;
    case 6: go.template operator()<6>(); break;
    default: go.template operator()<7>(); break;
  }
  return hipGetLastError();
}

hipError_t launch_dense_bwd_fast(int dtype, const DenseArgs& a, hipStream_t stream) {
  if (dtype == kBF16) return a.D == 64 ? launch_fast<bf16, 64>(a, stream) : launch_fast<bf16, 128>(a, stream);
  return a.D == 64 ? launch_fast<f16, 64>(a, stream) : launch_fast<f16, 128>(a, stream);
}

}  // namespace st
