// Gated dense block attention, forward: gfx950 path for 16-bit inputs with
// head_dim 64 or 128 (the hot shapes). Same algorithm as dense_fwd.hip
// (remote pass with one exp per score and block sums, remote mean parked in
// RC, then the local window pass); this variant
//  * runs two waves per SIMD in two phase-shifted groups (see the kernel),
//    so that one wave's MFMAs overlap the other's softmax;
//  * stages each 128-key K/V tile with asynchronous global->LDS copies into a
//    swizzled row-major layout, one group's copies during its softmax phase;
//  * reads K fragments with ds_read_b128 and V^T fragments with
//    ds_read_tr16_b64 (no transposed LDS stores), Q fragments from LDS in
//    register order;
//  * fixes the block size at compile time;
//  * numbers workgroups head-fastest so consecutive workgroups, which the
//    dispatcher spreads over the XCDs, keep one head's K/V per XCD L2.
#include <utility>

#include "dense.h"
#include "report.h"
#include "tile.h"

namespace st {

// Cost of splitting a row tile into two pieces, in key tiles: the second
// workgroup's dispatch, prologue (Q fragments, first K tile), epilogue (the
// two groups' join) and the merge kernel's share. Measured on cfg2's
// forward (with the merge) over 0..24 and "never": 12 is the fastest
// (76.5 us against 81.2 at 6, 84.9 at 0 and 82.1 never splitting).
constexpr int kPieceCost = 12;

// A work item is 128 query rows of one (batch, head), run by eight waves in
// two groups of four (one wave of each group per SIMD). Wave w owns rows
// 32(w%4)..+31 (lane = row on v_mfma_f32_32x32x16, score tiles transposed,
// S^T = K Q^T). Group 0 takes the first of the item's remote key tiles and
// then every local tile, group 1 the other remote tiles (counts balanced
// between the groups). Each
// group alternates MFMA phases (S^T products of its next tile, PV products
// of its previous one) with softmax phases, one workgroup barrier after
// each, and group 1 runs one phase behind group 0, so on every SIMD one
// wave's MFMAs overlap the other's softmax. A group stages its own K/V tiles
// (one buffer each) during its softmax phase. At the end group 1's partial
// remote state joins group 0's through LDS (the exact combination of two
// online-softmax states that dense_fwd_merge also uses).
template <typename T, int DP, int LOGB>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void dense_fwd_fast_kernel(DenseArgs a, int n_qtiles) {
  typedef Mma<T> M;
  typedef typename M::Frag Frag;
  constexpr int WAVES = 8;
  constexpr int NT = 128;
  constexpr int NST = NT / 32;
  constexpr int NDT = DP / 32;
  constexpr int NKC = DP / M::KW;
  constexpr int TILE = NT * DP;
  // The item's Q fragments (in register order: fragment c of lane l of the
  // waves owning rows 32w..32w+31 at 512 (4 c + w) + 8 l elements), then K
  // of group 0 and group 1, then V of group 0 and group 1: 160 KiB at head
  // dim 128. One LDS object (the per-lane fragment offsets below carry the
  // group's buffers, so every read is one address register plus an
  // immediate); the copies into a group's buffers are waited for before that
  // group's next reads anyway. The key-range table (before Q is stored) and
  // the epilogue's per-row statistics (after the last Q read) use the Q area.
  __shared__ __attribute__((aligned(16))) T kvs[5][TILE];
  int (*range)[4][WAVES] = reinterpret_cast<int (*)[4][WAVES]>(&kvs[0][0]);  // [2][4][WAVES]
  float (*xrow)[128] = reinterpret_cast<float (*)[128]>(&kvs[0][0]);         // [3][128]

  const int lane = threadIdx.x & 63;
  // wave-uniform (scalar): the group branches stay scalar branches
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2, wg = wave & 3;
  const int col = lane & 31, half = lane >> 5;
  const int BH = a.B * a.H;
  const int bh = blockIdx.x % BH, slot = blockIdx.x / BH;
  const int bi = bh / a.H, hh = bh % a.H;
  const int64_t H = a.H, D = a.D, N = a.N;
  constexpr int b = 1 << LOGB;

  // The job of this workgroup: row tile qt whole, or its piece `piece`.
  // Slot mode: f_pieces n_qtiles slots per head, slot k takes piece
  // k / n_qtiles of row tile n_qtiles-1-k % n_qtiles (longest causal rows
  // first; the pieces of an unsplit tile other than the first do nothing).
  // Pair mode: row tiles L = n-1-j and S = j form pair j; slot j
  // (j < n/2) takes L whole or its first piece, slot n/2+j takes S whole;
  // after an odd middle tile, slot 2(n/2)+odd+j takes L's second piece if L
  // is split, else nothing. L is split only where its second piece plus S,
  // plus the cost of the extra piece, stays below L whole; the second pieces
  // (longest first) then go to the compute units that finish S first.
  // Per lane: the row's remote limit and local window [llo, lhi] for row
  // tile qt.
  struct RowKeys {
    int64_t p;
    int rlim, llo, lhi;
  };
  auto row_keys = [&](int qt) -> RowKeys {
    const int row = qt * 128 + wg * 32 + col;
    RowKeys r = {row < a.Q ? a.pos[(int64_t)bi * a.Q + row] : -1, 0, 0, -1};
    if (r.p >= 0) {
      const int64_t c = r.p >> LOGB;
      const int64_t lo = (c - 1) * b > 0 ? (c - 1) * b : 0;
      r.rlim = (int)(lo < N ? lo : N);
      r.llo = (int)lo;
      r.lhi = (int)(r.p < N - 1 ? r.p : N - 1);
    }
    return r;
  };
  // Workgroup key ranges of a row tile (slot k of the LDS table): max
  // remote limit, min / max local key, min remote limit of the rows with a
  // local window; and from them the tile counts. publish_keys writes a
  // wave's part, collect_keys (after a barrier) combines the waves'.
  struct TileKeys {
    int n_remote_all, lt0, n_local, full_remote;
  };
  auto publish_keys = [&](const RowKeys& r, int k) {
    const bool win = r.lhi >= r.llo;
    const int r0 = wave_max(r.rlim), r1 = wave_min(win ? r.llo : 0x7fffffff);
    const int r2 = wave_max(win ? r.lhi : -1), r3 = wave_min(win ? r.rlim : 0x7fffffff);
    if (lane == 0) {
      range[k][0][wave] = r0;
      range[k][1][wave] = r1;
      range[k][2][wave] = r2;
      range[k][3][wave] = r3;
    }
  };
  auto collect_keys = [&](int k) -> TileKeys {
    int rg0 = range[k][0][0], rg1 = range[k][1][0], rg2 = range[k][2][0], rg3 = range[k][3][0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) {
      rg0 = max(rg0, range[k][0][w]);
      rg1 = min(rg1, range[k][1][w]);
      rg2 = max(rg2, range[k][2][w]);
      rg3 = min(rg3, range[k][3][w]);
    }
    rg0 = __builtin_amdgcn_readfirstlane(rg0);
    rg1 = __builtin_amdgcn_readfirstlane(rg1);
    rg2 = __builtin_amdgcn_readfirstlane(rg2);
    rg3 = __builtin_amdgcn_readfirstlane(rg3);
    TileKeys t;
    // remote tiles ending at or below every valid row's remote limit need
    // no masks (padding rows are zeroed when the row is finalised)
    t.full_remote = rg3 == 0x7fffffff ? 0 : rg3 / NT;
    t.n_remote_all = (rg0 + NT - 1) / NT;
    t.lt0 = rg2 >= 0 ? rg1 / NT : 0;
    t.n_local = rg2 >= 0 ? rg2 / NT - t.lt0 + 1 : 0;
    return t;
  };

  int qt, piece = 0;
  bool split = false;  // this job is a piece of a split row tile
  int hsplit = 0;      // remote tiles per piece (the last piece: the rest, and the local tiles)
  TileKeys tk;
  RowKeys rk;  // this lane's row of row tile qt
  const bool middle = a.f_pair && (n_qtiles & 1) && slot == 2 * (n_qtiles / 2);
  if (a.f_pair && !middle) {
    // pair j: both tiles' key ranges decide whether L is split (the same
    // decision in all three workgroups of the pair); a piece boundary
    // (second workgroup start, epilogue, merge) counts as kPieceCost tiles
    const int P = n_qtiles / 2, odd = n_qtiles & 1;
    const int j = slot < P ? slot : (slot < 2 * P ? slot - P : slot - 2 * P - odd);
    const int L = n_qtiles - 1 - j;
    // both row tiles' positions in flight together, one barrier
    const RowKeys rL = row_keys(L), rS = row_keys(j);
    publish_keys(rL, 0);
    publish_keys(rS, 1);
    __syncthreads();
    const TileKeys tl = collect_keys(0), ts = collect_keys(1);
    const int cL = tl.n_remote_all + tl.n_local, cS = ts.n_remote_all + ts.n_local;
    const int h = min(tl.n_remote_all, (cL + cS + kPieceCost + 1) / 2);
    const bool sp = a.fw0 != nullptr && h > 0 && h < cL && max(h, cL - h + cS + kPieceCost) < cL;
    if (slot < P) {
      qt = L;  // L whole, or its first piece
    } else if (slot < 2 * P) {
      qt = j;  // S whole
    } else {
      if (!sp) return;  // L ran whole
      qt = L;  // L's second piece
      piece = 1;
    }
    split = sp && qt == L;
    hsplit = h;
    tk = qt == L ? tl : ts;
    rk = qt == L ? rL : rS;
  } else {
    // slot mode: slot k takes piece k / n_qtiles of row tile
    // n_qtiles-1-k % n_qtiles (longest causal rows first); an odd middle
    // tile of pair mode runs whole
    if (a.f_pair) {
      qt = n_qtiles / 2;
    } else {
      piece = slot / n_qtiles;
      qt = n_qtiles - 1 - slot % n_qtiles;
    }
    rk = row_keys(qt);
    publish_keys(rk, 0);
    __syncthreads();
    tk = collect_keys(0);
    const int n_all = tk.n_remote_all + tk.n_local;
    if (a.fw0 != nullptr && !a.f_pair && n_all > a.f_split) {
      split = true;
      hsplit = (n_all + a.f_pieces - 1) / a.f_pieces;
    }
    if (piece > 0 && !split) return;  // whole workgroup
  }
  // pieces of this job's row tile (pair mode: two)
  const int n_pieces = split ? (a.f_pair ? 2 : a.f_pieces) : 1;
  const bool last_piece = piece == n_pieces - 1;
  const int row = qt * 128 + wg * 32 + col;
  const bool row_in = row < a.Q;
  const int64_t p = rk.p;
  const int rlim = rk.rlim, llo = rk.llo, lhi = rk.lhi;
  // (all of the tile bookkeeping below is workgroup-uniform: kept in SGPRs
  // so that the loop's branches are scalar)
  const int full_remote = __builtin_amdgcn_readfirstlane(tk.full_remote);
  const int n_remote_all = __builtin_amdgcn_readfirstlane(tk.n_remote_all);
  const int lt0 = __builtin_amdgcn_readfirstlane(tk.lt0), n_local = __builtin_amdgcn_readfirstlane(tk.n_local);
  // A split row tile runs as n_pieces pieces: piece p takes remote tiles
  // [p h, (p+1) h) (clipped to the remote range), the last piece the rest
  // of them and the local tiles; dense_fwd_merge combines their partial
  // results (a piece without tiles contributes nothing).
  if (!split) hsplit = n_remote_all;
  const int item = bh * n_qtiles + qt;
  const int rs = __builtin_amdgcn_readfirstlane(min(piece * hsplit, n_remote_all));  // first remote tile of this piece
  const int re = last_piece ? n_remote_all : min((piece + 1) * hsplit, n_remote_all);
  const int n_remote = __builtin_amdgcn_readfirstlane(re - rs);  // remote tiles of this piece
  const int n_loc = last_piece ? n_local : 0;  // local tiles of this piece
  if (split && n_remote == 0 && n_loc == 0) {
    // a piece without tiles (only a non-last piece can be one): its
    // statistics say "no mass", its mean is zero, and the first piece marks
    // the item as split
    const int lrow = wg * 32 + col;
    float* mean0 = a.fw0 + ((size_t)piece * BH * n_qtiles + bh * n_qtiles + qt) * 128 * D;
    for (int i = threadIdx.x; i < 128 * DP / 4; i += 512)
      if (qt * 128 + (4 * i) / DP < a.Q) reinterpret_cast<f32x4*>(mean0)[i] = f32x4{};
    if (grp == 0 && half == 0 && qt * 128 + lrow < a.Q) {
      float* st4 = a.fstat + ((size_t)(bh * n_qtiles + qt) * 128 + lrow) * 4 * (n_pieces + 1) + 4 * piece;
      st4[0] = kNegInf;
      st4[1] = 0.f;
      st4[2] = 0.f;
    }
    if (!piece && threadIdx.x == 0) a.fflag[bh * n_qtiles + qt] = 1;
    return;
  }
  // this group's tiles: group 0 the first r0 remote tiles, then the local
  // ones; group 1 the other remote tiles (r0 balances the two counts)
  const int r0 = __builtin_amdgcn_readfirstlane(min(n_remote, max(0, (n_remote - n_loc + 1) / 2)));
  const int my_remote = grp ? n_remote - r0 : r0;
  const int my_first = grp ? rs + r0 : rs;  // first remote tile of this group
  const int my_n = my_remote + (grp ? 0 : n_loc);
  auto tile_of = [&](int k) __attribute__((always_inline)) {
    return k < my_remote ? my_first + k : lt0 + (k - my_remote);
  };

  const T* kg = reinterpret_cast<const T*>(a.k) + ((int64_t)bi * N * H + hh) * D;
  const T* vg = reinterpret_cast<const T*>(a.v) + ((int64_t)bi * N * H + hh) * D;
  const int64_t kstride = H * D;
  // each group stages its own tiles
  const int gtid = (int)threadIdx.x & 255;
  const Stager<T, DP, 4> kst(kg, kstride, a.N, gtid), vst(vg, kstride, a.N, gtid);
  T* const lds = &kvs[0][0];
  T* const kbuf = lds + (1 + grp) * TILE;
  T* const vbuf = lds + (3 + grp) * TILE;
  // this lane's Q fragments: element offset of fragment c is qoff + 2048 c
  // (NKC fragments of 4 waves x 64 lanes x 8 elements fill the Q area)
  static_assert(NKC * 2048 == TILE, "Q fragments fill one tile");
  const int qoff = 512 * wg + 8 * lane;

  // Per-lane LDS fragment offsets (elements). The swizzle of a fragment row
  // depends only on the lane (tile row offsets are multiples of 16), so the
  // subtile parts of every address are compile-time immediates.
  int koff[NKC];
#pragma unroll
  for (int c = 0; c < NKC; ++c) koff[c] = (1 + grp) * TILE + col * DP + (((2 * c + half) ^ swz<DP>(col)) * 8);
  int voff[NDT], voff8[NDT];  // rows r0 and r0 + 8 (swizzled separately)
  {
    const int gi = lane >> 4, sl = lane & 15;
    const int r0 = 4 * (gi >> 1) + (sl >> 2);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d = 32 * dt + 16 * (gi & 1) + 4 * (sl & 3);
      voff[dt] = (3 + grp) * TILE + r0 * DP + (((d >> 3) ^ swz<DP>(r0)) * 8) + (d & 7);
      voff8[dt] = (3 + grp) * TILE + (r0 + 8) * DP + (((d >> 3) ^ swz<DP>(r0 + 8)) * 8) + (d & 7);
    }
  }
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef short s8 __attribute__((ext_vector_type(8)));
  // (fragments of this group's K and V tiles)
  auto kfrag = [&](int st, int c) __attribute__((always_inline)) -> Frag {
    return *reinterpret_cast<const Frag*>(lds + 32 * st * DP + koff[c]);
  };
  auto vfrag = [&](int k0, int dt) __attribute__((always_inline)) -> Frag {
    const T* p0 = lds + k0 * DP + voff[dt];
    const T* p1 = lds + k0 * DP + voff8[dt];
    s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)p0);
    s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)p1);
    return __builtin_bit_cast(Frag, (s8)__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  // PV accumulator (acc^T[d][row], lane = row): the remote pass, then (group
  // 0) the local pass
  f32x16 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc[dt] = zero16();
  const int64_t obase = (((int64_t)bi * a.Q + row) * H + hh) * D;
  // running state of the remote pass (max, row sum, sum of squared block
  // sums) and of the local pass (max, row sum); maxima in log2 units; the
  // sums are this lane's part (its half of the row's keys), joined with the
  // other half when the pass ends
  float m_r = kNegInf, zs_r = 0.f, dr = 0.f, m_l = kNegInf, zs_l = 0.f;

  // Group 0's end of the remote pass: join the halves of its sums and, when
  // local tiles follow, park its remote mean acc/dr in rc (one burst of
  // stores that drains while the local tiles run).
  const bool park_rc = last_piece;  // other pieces keep their remote sums for the epilogue
  auto finish_remote = [&]() __attribute__((always_inline)) {
    zs_r += swap_halves(zs_r);
    dr += swap_halves(dr);
    if (park_rc) {
      const float inv = dr > 0.f ? 1.f / dr : 0.f;
      if (row_in) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int d = 32 * dt + 8 * i + 4 * half;
            f32x4 val = {acc[dt][4 * i] * inv, acc[dt][4 * i + 1] * inv, acc[dt][4 * i + 2] * inv,
                         acc[dt][4 * i + 3] * inv};
            *reinterpret_cast<f32x4*>(a.rc + obase + d) = val;
          }
      }
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) acc[dt] = zero16();
    }
  };

  // scores of the group's current tile (S^T: keys x rows); after its
  // softmax phase, the probabilities, converted to 16-bit PV operands in the
  // next MFMA phase (where the vector unit is otherwise idle) before the next
  // S^T products overwrite them
  f32x16 sc[NST];
#pragma unroll
  for (int st = 0; st < NST; ++st) sc[st] = zero16();
  // per subtile: the factor the probabilities are multiplied by when they
  // become PV operands (remote blocks of 32+ keys: the block sum, applied
  // in the MFMA phase, whose vector unit is otherwise idle; else 1)
  float gate[NST];
#pragma unroll
  for (int st = 0; st < NST; ++st) gate[st] = 1.f;
  // the probabilities of the group's last tile as 16-bit PV operands
  // (subtile st, 16-key half c2), made at the end of its softmax phase:
  // with two waves per SIMD the other group's softmax keeps the vector unit
  // busy during an MFMA phase, so the conversions belong to the softmax
  // phase (phase 0 multiplies zeros)
  Frag pb[NST][2];
#pragma unroll
  for (int st = 0; st < NST; ++st) pb[st][0] = pb[st][1] = Frag{};

  // MFMA phase k: PV products of the group's tile k-1 (V in vbuf) first,
  // then the S^T products of its tile k (K in kbuf), in chunks of 4 with the
  // LDS reads of the next chunk issued one chunk ahead.
  constexpr int NPV = NST * 2 * NDT;  // PV products per tile (16 keys x 32 dims each)
  constexpr int NSP = NST * NKC;      // S^T products per tile
  // Phase 0 multiplies the zero probabilities by the zeroed V buffer, and
  // phase n's S^T products (of the group's last K tile again) are discarded:
  // one code path for every phase.
  auto mfma_phase = [&](int k) __attribute__((always_inline)) {
    auto pv_load = [&](int q) __attribute__((always_inline)) { return vfrag(16 * (q / NDT), q % NDT); };
    auto pv_mma = [&](int q, Frag f) __attribute__((always_inline)) {
      const int st = q / (2 * NDT), c2 = (q / NDT) & 1;
      acc[q % NDT] = M::mma(f, pb[st][c2], acc[q % NDT]);
    };
    // S^T products contraction chunk outermost (product j: chunk j / NST,
    // subtile j % NST), so each Q fragment is read once per phase
    // (the Q fragment of contraction chunk c is read with chunk c's K
    // fragments, one chunk ahead)
    auto s_load = [&](int j) __attribute__((always_inline)) { return kfrag(j % NST, j / NST); };
    auto s_mma = [&](int j, Frag f, Frag qc) __attribute__((always_inline)) {
      const int st = j % NST, c = j / NST;
      sc[st] = M::mma(f, qc, c == 0 ? zero16() : sc[st]);
    };
    static_assert(NST == 4, "one contraction chunk per MFMA chunk");
    mfma_chunks_shared<NPV + NSP, 4, NPV, NPV>(
        [&](int j) __attribute__((always_inline)) { return j < NPV ? pv_load(j) : s_load(j - NPV); },
        [&](int g) __attribute__((always_inline)) {
          return *reinterpret_cast<const Frag*>(lds + qoff + 2048 * (g - NPV / 4));
        },
        [&](int j, Frag f, Frag qc) __attribute__((always_inline)) {
          if (j < NPV) pv_mma(j, f);
          else s_mma(j - NPV, f, qc);
        });
    // group 0: the last remote PV products (tile my_remote - 1) are in
    if (grp == 0 && k == my_remote) finish_remote();
  };

  // Softmax phase of the group's tile k: masks, the row max (lazy
  // rescaling: the max only moves when some row of the wave exceeds it by
  // more than kLazyLog2), exponentials, the row and block sums, the gate
  // (remote tiles: each probability times its block's sum), the 16-bit
  // probabilities for PV, and the accumulator's rescale before the PV
  // products of tile k.
  auto softmax_phase = [&]<bool MASKED>(int k) __attribute__((always_inline)) {
    const bool remote = k < my_remote;
    const int kb = tile_of(k) * NT;
    if constexpr (MASKED) {
      // key of register r in subtile st: kb + 4*half + 32*st + 8*(r/4) + r%4;
      // visible iff lo <= offset < lim (one unsigned compare)
      const int base = kb + 4 * half;
      const int lim = (remote ? rlim : lhi + 1) - base;
      const int lo = remote ? -(1 << 30) : llo - base;
      const uint32_t span = lim > lo ? (uint32_t)(lim - lo) : 0u;
#pragma unroll
      for (int st = 0; st < NST; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int off = 32 * st + 8 * (r >> 2) + (r & 3);
          sc[st][r] = (uint32_t)(off - lo) < span ? sc[st][r] : kNegInf;
        }
    }
    // balanced trees (short dependency chains)
    float mx4[NST];
#pragma unroll
    for (int st = 0; st < NST; ++st) mx4[st] = tree16<OpMax>(sc[st]);
    float mt = fmaxf(fmaxf(mx4[0], mx4[1]), fmaxf(mx4[2], mx4[3]));
    mt = fmaxf(mt, swap_halves(mt)) * a.scale_log2;
    const float m = remote ? m_r : m_l;
    const bool grow = __builtin_amdgcn_ballot_w64(mt > m + kLazyLog2) != 0;
    const float mn = grow ? fmaxf(m, mt) : m;
    const float msafe = mn == kNegInf ? 0.f : mn;
    const float alpha = fast_exp2(m - msafe);
    if (remote) m_r = mn;
    else m_l = mn;
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[st][r] = fast_exp2(fmaf(sc[st][r], a.scale_log2, -msafe));
    // in-lane sums per subtile, and the lane's part of the row sum
    float ps[NST];
#pragma unroll
    for (int st = 0; st < NST; ++st) ps[st] = tree16<OpAdd>(sc[st]);
    const float psum = (ps[0] + ps[1]) + (ps[2] + ps[3]);
    if (remote) {
      zs_r = zs_r * alpha + psum;
      if constexpr (LOGB >= 5) {
        // blocks of whole subtiles: block totals from the subtile sums
        constexpr int G = (1 << LOGB) / 32;
        float blk[NST];
        float w = 0.f;
#pragma unroll
        for (int g0 = 0; g0 < NST; g0 += G) {
          float part = ps[g0];
#pragma unroll
          for (int g = 1; g < G; ++g) part += ps[g0 + g];
          const float tot = part + swap_halves(part);
          w += part * tot;  // this lane's keys of the block times the block sum
#pragma unroll
          for (int g = 0; g < G; ++g) blk[g0 + g] = tot;
        }
        dr = dr * (alpha * alpha) + w;
#pragma unroll
        for (int st = 0; st < NST; ++st) gate[st] = blk[st];  // applied in the MFMA phase
      } else {
        float blkv[NST][8];
        block_sums<NST, LOGB>(sc, blkv);
        float w = 0.f;
#pragma unroll
        for (int st = 0; st < NST; ++st)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            sc[st][r] *= blkv[st][blk_slot<LOGB>(r)];
            w += sc[st][r];
          }
        dr = dr * (alpha * alpha) + w;
      }
    } else {
      zs_l = zs_l * alpha + psum;
    }
    if constexpr (LOGB >= 5) {
      if (!remote) {
#pragma unroll
        for (int st = 0; st < NST; ++st) gate[st] = 1.f;
      }
    }
    if (grow) {
      // acc holds the sums of earlier tiles at the old max (squared for the
      // remote pass, whose weights carry two factors of 2^-m)
      const float f = remote ? alpha * alpha : alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) acc[dt] *= f;
    }
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
        for (int e = 0; e < 8; ++e) pb[st][c2][e] = from_float<T>(sc[st][8 * c2 + e] * gate[st]);
  };

  // Phases: MFMA(0), softmax(0), MFMA(1), ..., softmax(n-1), MFMA(n) for the
  // group's n tiles, a barrier after each; group 1 starts one barrier later,
  // and both groups end on the same barrier count. During softmax(k) the
  // group stages K of its tile k+1 and V of its tile k (MFMA(k) has read the
  // previous contents) and waits for the copies before the barrier.
  const int my_bars = grp ? 2 * my_n + 2 : 2 * my_n + 1;
  const int n0 = r0 + n_loc, n1 = n_remote - r0;
  const int all_bars = __builtin_amdgcn_readfirstlane(max(2 * n0 + 1, 2 * n1 + 2));
  __syncthreads();  // the key-range table in the Q area is read
  if (grp == 0) {
    // Q fragments of this wave's rows (the B operands of S^T = K Q^T)
    const T* qrow = reinterpret_cast<const T*>(a.q) + (((int64_t)bi * a.Q + (row_in ? row : 0)) * H + hh) * D;
#pragma unroll
    for (int c = 0; c < NKC; ++c)
      *reinterpret_cast<Frag*>(lds + qoff + 2048 * c) =
          row_in ? *reinterpret_cast<const Frag*>(qrow + c * 16 + half * 8) : Frag{};
  }
  if (my_n > 0) kst.template stage<NT>(kbuf, tile_of(0) * NT);
  {
    // zero V buffer for phase 0's PV products (16 bytes per thread and pass)
    typedef typename Vec16<T>::type V;
    V* z = reinterpret_cast<V*>(vbuf);
#pragma unroll
    for (int i = gtid; i < TILE / Vec16<T>::n; i += 256) z[i] = V{};
  }
  wait_vm();
  __syncthreads();
  if (grp == 1) __syncthreads();
  auto step = [&]<bool MASKED>(int k) __attribute__((always_inline)) {
    mfma_phase(k);
    __syncthreads();
    if (k < my_n) {
      if (k + 1 < my_n) kst.template stage<NT>(kbuf, tile_of(k + 1) * NT);
      vst.template stage<NT>(vbuf, tile_of(k) * NT);
      softmax_phase.template operator()<MASKED>(k);
      wait_vm();
      __syncthreads();
    }
  };
  // the group's unmasked tiles (remote tiles below every row's remote
  // limit) come first: one loop per softmax variant
  const int n_fast = __builtin_amdgcn_readfirstlane(min(my_remote, max(0, full_remote - my_first)));
  int k = 0;
  for (; k < n_fast; ++k) step.template operator()<false>(k);
  for (; k <= my_n; ++k) step.template operator()<true>(k);
  for (int i = my_bars; i < all_bars; ++i) __syncthreads();

  // Epilogue. Every wave has passed the last barrier: the K/V buffers are
  // free. Group 1 stages its remote mean (acc/dr, lane = row) and its
  // statistics; group 0 joins them with its own state and writes the item's
  // results (or the piece's partials for dense_fwd_merge) row-contiguously.
  constexpr int CM = DP / 4 - 1;  // 16-byte chunks of a staged fp32 row, swizzled by the row
  auto sidx = [](int r, int d) __attribute__((always_inline)) { return r * DP + ((((d >> 2) ^ (r & CM)) << 2) | (d & 3)); };
  static_assert(2 * 32 * DP * 4 <= TILE * (int)sizeof(T), "two waves' rows fit one buffer");
  float* stage1 = reinterpret_cast<float*>(kvs[1 + (wg >> 1)]) + (wg & 1) * 32 * DP;  // group 1's rows of wave wg
  float* stage0 = reinterpret_cast<float*>(kvs[3 + (wg >> 1)]) + (wg & 1) * 32 * DP;  // group 0's rows of wave wg
  auto stage_acc = [&](float* dst, float f) __attribute__((always_inline)) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 32 * dt + 8 * i + 4 * half;
        const f32x4 v = {acc[dt][4 * i] * f, acc[dt][4 * i + 1] * f, acc[dt][4 * i + 2] * f, acc[dt][4 * i + 3] * f};
        *reinterpret_cast<f32x4*>(dst + sidx(col, d)) = v;
      }
  };
  const int lrow = wg * 32 + col;  // row within the item
  if (grp == 1) {
    zs_r += swap_halves(zs_r);
    dr += swap_halves(dr);
    stage_acc(stage1, dr > 0.f ? 1.f / dr : 0.f);
    if (half == 0) {
      xrow[0][lrow] = m_r;
      xrow[1][lrow] = zs_r;
      xrow[2][lrow] = dr;
    }
  }
  __syncthreads();
  if (grp == 1) return;
  // the two remote states at their common max (dense_fwd_merge's
  // combination): weights dr_g 2^{2(m_g - m)} of the groups' means
  const float m1 = xrow[0][lrow], zs1 = xrow[1][lrow], dr1 = xrow[2][lrow];
  const float mx = fmaxf(m_r, m1);
  float zs = 0.f, w0 = 0.f, w1 = 0.f;
  if (mx != kNegInf) {
    const float e0 = fast_exp2(m_r - mx), e1 = fast_exp2(m1 - mx);
    zs = zs_r * e0 + zs1 * e1;
    w0 = dr * e0 * e0;
    w1 = dr1 * e1 * e1;
  }
  const float drs = w0 + w1;
  const float a0 = drs > 0.f ? w0 / drs : 0.f, a1 = drs > 0.f ? w1 / drs : 0.f;
  float log_zr = zs > 0.f ? log_mass(mx, zs) : kNegInf;
  float lr = drs > 0.f ? log_mass(mx, drs) - fast_log2(zs) * kLn2 : kNegInf;
  const float zsum = zs_l + swap_halves(zs_l);
  constexpr int RL = DP / 4;          // lanes per row, 4 floats each
  constexpr int NIT = 32 * RL / 64;   // row-contiguous passes over the wave's 32 rows
  const int row0 = qt * 128 + wg * 32;
  if (a.fw0 != nullptr && !piece && threadIdx.x == 0) a.fflag[item] = split ? 1 : 0;
  float xa0, xa1;  // per row: weights of the two remote means in the written remote part
  float sf;        // scale of the staged acc
  // this row's partial statistics: (max, row sum, sum of squared block
  // sums) of piece p at 4 p, the local (max, row sum) at 4 n_pieces
  float* st4 = a.fstat + ((size_t)item * 128 + lrow) * 4 * (n_pieces + 1);
  if (split && !last_piece) {
    // partial of a piece without local tiles: the joined remote mean
    xa0 = 0.f;
    xa1 = a1;
    sf = dr > 0.f ? a0 / dr : 0.f;  // acc holds group 0's unnormalised remote sums
    if (half == 0 && row_in) {
      st4[4 * piece] = mx; st4[4 * piece + 1] = zs; st4[4 * piece + 2] = drs;
    }
  } else if (split) {
    // partial of the last piece: the joined remote mean (rc) and the local mean
    xa0 = a0;
    xa1 = a1;
    sf = zsum > 0.f ? 1.f / zsum : 0.f;
    if (half == 0 && row_in) {
      st4[4 * piece] = mx; st4[4 * piece + 1] = zs; st4[4 * piece + 2] = drs;
      st4[4 * n_pieces] = m_l; st4[4 * n_pieces + 1] = zsum;
    }
  } else {
    const float dl = p >= 0 ? zsum : 0.f;
    const float ll = p >= 0 ? log_mass(m_l, dl) : kNegInf;
    if (p < 0) {
      lr = kNegInf;
      log_zr = kNegInf;
    }
    const float tot = logaddexp(lr, ll);
    const float safe_total = tot == kNegInf ? 0.f : tot;
    const float prem = lr == kNegInf ? 0.f : __expf(lr - safe_total);
    const float ploc = ll == kNegInf ? 0.f : __expf(ll - safe_total);
    xa0 = prem * a0;
    xa1 = prem * a1;
    sf = dl > 0.f ? ploc / dl : 0.f;
    if (half == 0 && row_in) {
      const int64_t si = ((int64_t)bi * a.Q + row) * H + hh;
      a.pr[si] = prem;
      a.zr[si] = log_zr;
      a.z[si] = tot;
    }
  }
  stage_acc(stage0, sf);
  if (half == 0) {
    xrow[0][lrow] = xa0;
    xrow[1][lrow] = xa1;
  }
  // this wave's staged rows and weights (and its parked rc stores) are
  // visible to all its lanes
  __threadfence_block();
  __builtin_amdgcn_wave_barrier();
  typedef T T4 __attribute__((ext_vector_type(4)));
  const int mode = split ? (last_piece ? 1 : 0) : 2;
  const size_t n_items = (size_t)BH * n_qtiles;
  float* fdst = split ? (last_piece ? a.fw1 + (size_t)item * 128 * D
                                    : a.fw0 + ((size_t)piece * n_items + item) * 128 * D)
                      : nullptr;
  // every global load before the first store (the stores may alias in the
  // compiler's view, which would serialise the round trips)
  f32x4 mean[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int r = (it * 64 + lane) / RL, c = ((it * 64 + lane) % RL) * 4;
    const int64_t gi = (((int64_t)bi * a.Q + row0 + r) * H + hh) * D + c;
    mean[it] = (mode != 0 && row0 + r < a.Q) ? *reinterpret_cast<const f32x4*>(a.rc + gi) : f32x4{};
  }
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int r = (it * 64 + lane) / RL, c = ((it * 64 + lane) % RL) * 4;
    if (row0 + r >= a.Q) continue;
    const int64_t gi = (((int64_t)bi * a.Q + row0 + r) * H + hh) * D + c;
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(stage0 + sidx(r, c));
    const f32x4 s1 = *reinterpret_cast<const f32x4*>(stage1 + sidx(r, c));
    const float x0 = xrow[0][wg * 32 + r], x1 = xrow[1][wg * 32 + r];
    const f32x4 rem = mean[it] * x0 + s1 * x1;  // the remote part (piece 0: group 1's share)
    if (mode == 0) {
      *reinterpret_cast<f32x4*>(fdst + (int64_t)(wg * 32 + r) * D + c) = s0 + rem;
    } else if (mode == 1) {
      *reinterpret_cast<f32x4*>(a.rc + gi) = rem;
      *reinterpret_cast<f32x4*>(fdst + (int64_t)(wg * 32 + r) * D + c) = s0;
    } else {
      T4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = from_float<T>(rem[j] + s0[j]);
      *reinterpret_cast<f32x4*>(a.rc + gi) = rem;
      *reinterpret_cast<T4*>(reinterpret_cast<T*>(a.out) + gi) = o;
    }
  }
}

// Combination of the pieces of every split row tile: the remote partials
// (per piece: max m, row sum zs, sum of squared block sums dr, all at scale
// 2^-m, and the remote mean) merged at the common max, then the gate with
// the local partial of the last piece as in the single-piece epilogue. DP/8
// threads per row, 8 values each: every access is row-contiguous, and all
// loads of a thread are issued before its arithmetic.
template <typename T, int DP, int P>
__global__ __launch_bounds__(256) void dense_fwd_merge_kernel(DenseArgs a, int n_qtiles) {
  constexpr int TR = DP / 8;      // threads per row
  constexpr int RPW = 256 / TR;   // rows per workgroup
  constexpr int WPI = 128 / RPW;  // workgroups per row tile
  const int item = blockIdx.x / WPI;
  if (a.fflag[item] == 0) return;
  const int bh = item / n_qtiles, qt = item % n_qtiles;
  const int bi = bh / a.H, hh = bh % a.H;
  const int lrow = (blockIdx.x % WPI) * RPW + threadIdx.x / TR, row = qt * 128 + lrow;
  if (row >= a.Q) return;
  const int c = (threadIdx.x % TR) * 8;
  const int64_t H = a.H, D = a.D;
  const int64_t g = (((int64_t)bi * a.Q + row) * H + hh) * D + c;
  const size_t w = ((size_t)item * 128 + lrow) * D + c;
  const size_t piece_stride = (size_t)a.B * a.H * n_qtiles * 128 * D;
  const float* st4 = a.fstat + ((size_t)item * 128 + lrow) * 4 * (P + 1);
  const int64_t p = a.pos[(int64_t)bi * a.Q + row];
  f32x4 stat[P + 1], mean[P][2], meanl[2];
#pragma unroll
  for (int i = 0; i <= P; ++i) stat[i] = *reinterpret_cast<const f32x4*>(st4 + 4 * i);
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const float* src = i < P - 1 ? a.fw0 + i * piece_stride + w : a.rc + g;
    mean[i][0] = *reinterpret_cast<const f32x4*>(src);
    mean[i][1] = *reinterpret_cast<const f32x4*>(src + 4);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) meanl[h] = *reinterpret_cast<const f32x4*>(a.fw1 + w + 4 * h);
  float mx = kNegInf;
#pragma unroll
  for (int i = 0; i < P; ++i) mx = fmaxf(mx, stat[i][0]);
  float zs = 0.f, drs = 0.f, wt[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const float e = mx != kNegInf ? fast_exp2(stat[i][0] - mx) : 0.f;
    zs += stat[i][1] * e;
    wt[i] = stat[i][2] * e * e;
    drs += wt[i];
  }
  const float m_loc = stat[P][0], zl = stat[P][1];
  float log_zr = zs > 0.f ? log_mass(mx, zs) : kNegInf;
  float lr = drs > 0.f ? log_mass(mx, drs) - fast_log2(zs) * kLn2 : kNegInf;
  float ll = zl > 0.f ? log_mass(m_loc, zl) : kNegInf;
  if (p < 0) { lr = kNegInf; ll = kNegInf; log_zr = kNegInf; }
  const float tot = logaddexp(lr, ll);
  const float safe_total = tot == kNegInf ? 0.f : tot;
  const float prem = lr == kNegInf ? 0.f : __expf(lr - safe_total);
  const float ploc = ll == kNegInf ? 0.f : __expf(ll - safe_total);
  const float f = drs > 0.f ? prem / drs : 0.f;
  typedef T T8 __attribute__((ext_vector_type(8)));
  T8 o;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    // (a piece without mass has weight 0: selected away, not multiplied)
    f32x4 rc = {};
#pragma unroll
    for (int i = 0; i < P; ++i)
      if (wt[i] > 0.f) rc += mean[i][h] * (wt[i] * f);
    *reinterpret_cast<f32x4*>(a.rc + g + 4 * h) = rc;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[4 * h + j] = from_float<T>(rc[j] + ploc * meanl[h][j]);
  }
  *reinterpret_cast<T8*>(reinterpret_cast<T*>(a.out) + g) = o;
  if (c == 0) {
    const int64_t sidx = ((int64_t)bi * a.Q + row) * H + hh;
    a.pr[sidx] = prem;
    a.zr[sidx] = log_zr;
    a.z[sidx] = tot;
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
  const unsigned items = (unsigned)(n_qtiles * a.B * a.H);
  // pair mode (two pieces) once slot mode's two-piece slots outnumber the
  // compute units; else slot mode with the workspace's piece count (more
  // than two for launches with few row tiles)
  a.f_pair = a.fw0 != nullptr && 2 * (int64_t)items > device_cus();
  if (a.f_pair) a.f_pieces = 2;
  const int per_head = a.f_pair ? 3 * (n_qtiles / 2) + (n_qtiles & 1) : a.fw0 != nullptr ? a.f_pieces * n_qtiles : n_qtiles;
  dim3 grid((unsigned)(per_head * a.B * a.H));
  auto go = [&]<int LOGB>() {
    note_launch((const void*)&dense_fwd_fast_kernel<T, DP, LOGB>,
                {"dense_fwd_fast", dtype_code<T>(), DP, 1 << LOGB, 128, 128, 8, 2, grid.x,
                 a.f_pair ? "pair" : (a.fw0 ? "slot" : "grid")});
    hipLaunchKernelGGL((dense_fwd_fast_kernel<T, DP, LOGB>), grid, dim3(512), 0, stream, a, n_qtiles);
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
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.fw0 == nullptr) return e;
  constexpr int WPI = 128 / (256 / (DP / 8));
  auto merge = [&]<int P>() {
    note_launch((const void*)&dense_fwd_merge_kernel<T, DP, P>,
                {"dense_fwd_merge", dtype_code<T>(), DP, a.block, 256 / (DP / 8), DP, 4, 0, items * WPI, "rows"});
    hipLaunchKernelGGL((dense_fwd_merge_kernel<T, DP, P>), dim3(items * WPI), dim3(256), 0, stream, a, n_qtiles);
  };
  if (a.f_pieces == 8) merge.template operator()<8>();
  else if (a.f_pieces == 4) merge.template operator()<4>();
  else merge.template operator()<2>();
  return hipGetLastError();
}

namespace {
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
}  // namespace

DenseFwdPlan dense_fwd_plan(int dtype, int64_t B, int64_t Q, int64_t N, int64_t H, int64_t D) {
  DenseFwdPlan p = {};
  p.fast = (dtype == kBF16 || dtype == kF16) && (D == 64 || D == 128) && N * H * D * 2 < (int64_t(1) << 31);
  if (!p.fast) return p;
  p.n_qtiles = (int)((Q + 127) / 128);
  const int64_t n_ktiles = (N + 127) / 128;
  if (n_ktiles < 4) return p;  // no row tile long enough to split: no workspace
  const size_t items = (size_t)(B * H) * p.n_qtiles;
  p.pieces = split_pieces((int64_t)items);
  const size_t w = align256(items * 128 * (size_t)D * sizeof(float));
  p.off_w1 = (p.pieces - 1) * w;
  p.off_stat = p.pieces * w;
  p.off_flag = p.off_stat + align256(items * 128 * 4 * (p.pieces + 1) * sizeof(float));
  p.total = p.off_flag + align256(items * sizeof(int));
  return p;
}

bool dense_fwd_fast_supported(int dtype, const DenseArgs& a) {
  // 32-bit buffer offsets within one batch's K/V
  return (dtype == kBF16 || dtype == kF16) && (a.D == 64 || a.D == 128) &&
         (int64_t)a.N * a.H * a.D * 2 < (int64_t(1) << 31);
}

hipError_t launch_dense_fwd_fast(int dtype, const DenseArgs& a, hipStream_t stream) {
  if (dtype == kBF16) return a.D == 64 ? launch_fast<bf16, 64>(a, stream) : launch_fast<bf16, 128>(a, stream);
  return a.D == 64 ? launch_fast<f16, 64>(a, stream) : launch_fast<f16, 128>(a, stream);
}

}  // namespace st
