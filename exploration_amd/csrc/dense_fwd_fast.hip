// Gated dense block attention, forward: pipelined gfx950 path for 16-bit
// inputs with head_dim 64 or 128 (the hot shapes). Same algorithm as
// dense_fwd.hip (remote pass with one exp per score and block sums, remote
// mean parked in RC, then the local window pass); this variant
//  * stages each 128-key K/V tile with asynchronous global->LDS copies into a
//    swizzled row-major layout, double-buffered so the copies of tile i+1
//    overlap the arithmetic of tile i;
//  * reads K fragments with ds_read_b128 and V^T fragments with
//    ds_read_tr16_b64 (no transposed LDS stores);
//  * fixes the block size at compile time;
//  * numbers workgroups head-fastest so consecutive workgroups, which the
//    dispatcher spreads over the XCDs, keep one head's K/V per XCD L2.
#include <utility>

#include "dense.h"
#include "report.h"
#include "tile.h"

namespace st {

// Cost of splitting a row tile into two pieces, in key tiles (~2.8 us each
// at D=128): the second workgroup's dispatch, prologue, first (cold) tiles
// and epilogue, and the merge. Measured on cfg2 over 1..8 and "never": 6 is
// the fastest (78 us against 88 at 3 and 98 never splitting).
constexpr int kPieceCost = 6;

template <typename T, int DP, int LOGB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void dense_fwd_fast_kernel(DenseArgs a, int n_qtiles) {
  typedef Mma<T> M;
  typedef typename M::Frag Frag;
  constexpr int WAVES = 4;
  constexpr int NT = 128;
  constexpr int NST = NT / 32;
  constexpr int NDT = DP / 32;
  constexpr int NKC = DP / M::KW;
  constexpr int TILE = NT * DP;
  // Two K and two V buffers as distinct LDS objects, selected at compile
  // time, so the compiler can tell the copies into one buffer from the reads
  // of the other and does not wait for the copies before reading.
  __shared__ __attribute__((aligned(16))) T k0s[TILE];
  __shared__ __attribute__((aligned(16))) T k1s[TILE];
  __shared__ __attribute__((aligned(16))) T v0s[TILE];
  __shared__ __attribute__((aligned(16))) T v1s[TILE];
  __shared__ int range[2][4][WAVES];  // two tiles: this one and the pair partner

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int BH = a.B * a.H;
  const int bh = blockIdx.x % BH, slot = blockIdx.x / BH;
  const int bi = bh / a.H, hh = bh % a.H;
  const int64_t H = a.H, D = a.D, N = a.N;
  constexpr int b = 1 << LOGB;

  // The job of this workgroup: row tile qt, kind 0 (the tile whole or its
  // first piece), 1 (its second piece; nothing if unsplit) or 2 (whole).
  // Slot mode: 2 n_qtiles slots per head, slot k < n_qtiles takes kind 0 of
  // row tile n_qtiles-1-k, slot n_qtiles+k kind 1 of it (longest causal rows
  // first). Pair mode: row tiles L = n-1-j and S = j form pair j; slot j
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
    const int row = qt * 32 * WAVES + wave * 32 + col;
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
  // Workgroup key ranges of a row tile (slot k of the LDS table; one barrier):
  // max remote limit, min / max local key, min remote limit of the rows with
  // a local window; and from them the tile counts.
  struct TileKeys {
    int n_remote_all, lt0, n_local, full_remote;
  };
  auto tile_keys = [&](const RowKeys& r, int k) -> TileKeys {
    const bool win = r.lhi >= r.llo;
    const int r0 = wave_max(r.rlim), r1 = wave_min(win ? r.llo : 0x7fffffff);
    const int r2 = wave_max(win ? r.lhi : -1), r3 = wave_min(win ? r.rlim : 0x7fffffff);
    if (lane == 0) {
      range[k][0][wave] = r0;
      range[k][1][wave] = r1;
      range[k][2][wave] = r2;
      range[k][3][wave] = r3;
    }
    __syncthreads();
    int rg0 = range[k][0][0], rg1 = range[k][1][0], rg2 = range[k][2][0], rg3 = range[k][3][0];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) {
      rg0 = max(rg0, range[k][0][w]);
      rg1 = min(rg1, range[k][1][w]);
      rg2 = max(rg2, range[k][2][w]);
      rg3 = min(rg3, range[k][3][w]);
    }
    // uniform by construction; in SGPRs, everything derived from them (tile
    // indices, loop bounds, staging addresses) stays scalar
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

  int qt, kind;
  bool split = false;  // this job is a piece of a split row tile
  int hsplit = 0;      // remote tiles of a split tile's first piece
  TileKeys tk;
  const bool middle = a.f_pair && (n_qtiles & 1) && slot == 2 * (n_qtiles / 2);
  if (a.f_pair && !middle) {
    // pair j: both tiles' key ranges decide whether L is split (the same
    // decision in all three workgroups of the pair); a piece boundary
    // (second workgroup start, epilogue, merge) counts as kPieceCost tiles
    const int P = n_qtiles / 2, odd = n_qtiles & 1;
    const int j = slot < P ? slot : (slot < 2 * P ? slot - P : slot - 2 * P - odd);
    const int L = n_qtiles - 1 - j;
    const TileKeys tl = tile_keys(row_keys(L), 0), ts = tile_keys(row_keys(j), 1);
    const int cL = tl.n_remote_all + tl.n_local, cS = ts.n_remote_all + ts.n_local;
    const int h = min(tl.n_remote_all, (cL + cS + kPieceCost + 1) / 2);
    const bool sp = a.fw0 != nullptr && h > 0 && h < cL && max(h, cL - h + cS + kPieceCost) < cL;
    if (slot < P) {
      qt = L;  // L whole, or its first piece
      kind = 0;
    } else if (slot < 2 * P) {
      qt = j;  // S whole
      kind = 2;
    } else {
      if (!sp) return;  // L ran whole
      qt = L;  // L's second piece
      kind = 1;
    }
    split = sp && qt == L;
    hsplit = h;
    tk = qt == L ? tl : ts;
  } else {
    if (a.f_pair) {
      qt = n_qtiles / 2;  // odd middle tile
      kind = 2;
    } else {
      kind = slot >= n_qtiles;
      qt = n_qtiles - 1 - (kind ? slot - n_qtiles : slot);
    }
    tk = tile_keys(row_keys(qt), 0);
    const int n_all = tk.n_remote_all + tk.n_local;
    if (a.fw0 != nullptr && kind != 2 && n_all > a.f_split) {
      split = true;
      hsplit = min((n_all + 1) / 2, tk.n_remote_all);
    }
    if (kind == 1 && !split) return;  // whole workgroup
  }
  const int row = qt * 32 * WAVES + wave * 32 + col;
  const bool row_in = row < a.Q;
  const RowKeys rk = row_keys(qt);
  const int64_t p = rk.p;
  const int rlim = rk.rlim, llo = rk.llo, lhi = rk.lhi;
  const int full_remote = tk.full_remote, n_remote_all = tk.n_remote_all, lt0 = tk.lt0, n_local = tk.n_local;
  // A split row tile runs as two pieces: piece 0 takes remote tiles [0, h),
  // piece 1 remote tiles [h, n_remote_all) and the local tiles;
  // dense_fwd_merge combines their partial results.
  if (!split) hsplit = n_remote_all;
  const int piece = kind == 1;
  const int item = bh * n_qtiles + qt;
  const int rs = piece ? hsplit : 0;                              // first remote tile of this piece
  const int n_remote = piece ? n_remote_all - hsplit : hsplit;    // remote tiles of this piece
  const bool with_local = !split || piece;
  const int total = n_remote + (with_local ? n_local : 0);
  auto tile_of = [&](int i) { return i < n_remote ? rs + i : lt0 + (i - n_remote); };

  const T* kg = reinterpret_cast<const T*>(a.k) + ((int64_t)bi * N * H + hh) * D;
  const T* vg = reinterpret_cast<const T*>(a.v) + ((int64_t)bi * N * H + hh) * D;
  const int64_t kstride = H * D;
  const Stager<T, DP, WAVES> kst(kg, kstride, a.N), vst(vg, kstride, a.N);

  Frag qf[NKC];
  {
    const T* qrow = reinterpret_cast<const T*>(a.q) + (((int64_t)bi * a.Q + (row_in ? row : 0)) * H + hh) * D;
#pragma unroll
    for (int c = 0; c < NKC; ++c) qf[c] = row_in ? *reinterpret_cast<const Frag*>(qrow + c * 16 + half * 8) : Frag{};
  }

  // Per-lane LDS fragment offsets (elements). The swizzle of a fragment row
  // depends only on the lane (tile row offsets are multiples of 16), so the
  // subtile and buffer parts of every address are compile-time immediates.
  int koff[NKC];
#pragma unroll
  for (int c = 0; c < NKC; ++c) koff[c] = col * DP + (((2 * c + half) ^ swz<DP>(col)) * 8);
  int voff[NDT], voff8[NDT];  // rows r0 and r0 + 8 (swizzled separately)
  {
    const int gi = lane >> 4, sl = lane & 15;
    const int r0 = 4 * (gi >> 1) + (sl >> 2);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d = 32 * dt + 16 * (gi & 1) + 4 * (sl & 3);
      voff[dt] = r0 * DP + (((d >> 3) ^ swz<DP>(r0)) * 8) + (d & 7);
      voff8[dt] = (r0 + 8) * DP + (((d >> 3) ^ swz<DP>(r0 + 8)) * 8) + (d & 7);
    }
  }
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef short s8 __attribute__((ext_vector_type(8)));
  auto kfrag = [&](const T* buf, int st, int c) -> Frag {
    return *reinterpret_cast<const Frag*>(buf + 32 * st * DP + koff[c]);
  };
  auto vfrag = [&](const T* buf, int k0, int dt) -> Frag {
    const T* p0 = buf + k0 * DP + voff[dt];
    const T* p1 = buf + k0 * DP + voff8[dt];
    s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)p0);
    s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)p1);
    return __builtin_bit_cast(Frag, (s8)__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  // PV accumulator (acc^T[d][row], lane = row): the remote pass, then the
  // local pass
  f32x16 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc[dt] = zero16();
  const int64_t obase = (((int64_t)bi * a.Q + row) * H + hh) * D;
  // running state of the remote pass (max, row sum, sum of squared block
  // sums) and of the local pass (max, row sum); maxima in log2 units
  float m_r = kNegInf, zs_r = 0.f, dr = 0.f, m_l = kNegInf, zs_l = 0.f;
  float log_zr = kNegInf, lr = kNegInf;

  // End of the remote pass: its statistics, and its mean parked in rc (one
  // burst of stores that drains while the local tiles run; registers cannot
  // hold two accumulators next to the pipelined loop).
  const bool park_rc = !(split && piece == 0);  // piece 0 writes its mean in the epilogue
  auto finish_remote = [&]() {
    zs_r += swap_halves(zs_r);
    dr += swap_halves(dr);
    log_zr = log_mass(m_r, zs_r);
    lr = dr > 0.f ? log_mass(m_r, dr) - fast_log2(zs_r) * kLn2 : kNegInf;
    const float inv = dr > 0.f ? 1.f / dr : 0.f;
    if (row_in && park_rc) {
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
    // the local pass starts from zero; piece 0 keeps its remote sums for
    // the epilogue
    if (park_rc) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) acc[dt] = zero16();
    }
  };

  // Software pipeline over the tile sequence. Iteration i issues, in one
  // scheduling region, the PV MFMAs of tile i-1 (V buffer (i+1)&1) while the
  // VALU masks, maximises and exponentiates the scores of tile i, then the
  // S^T MFMAs of tile i+1 (K buffer (i+1)&1) while the VALU scales and
  // converts tile i to 16-bit probabilities; the S^T products of subtile st
  // overwrite scores the softmax has finished with, so one score buffer and
  // one probability buffer suffice. Products go in chunks of 4 with their LDS
  // reads one chunk ahead. Past the ends of the sequence the MFMAs run on
  // finite filler data whose results are never used (probabilities of tile
  // -1 are zero; scores of tile `total` are discarded).
  f32x16 sc[NST];
  Frag pf[NST][2];
#pragma unroll
  for (int st = 0; st < NST; ++st)
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) pf[st][c2] = Frag{};
  constexpr int NSP = NST * NKC;      // S^T products per tile
  constexpr int NPV = NST * 2 * NDT;  // PV products per tile
  constexpr int H1 = NPV / 4;         // chunks of the first half (PV)
  constexpr int H2 = NSP / 4;         // chunks of the second half (S^T)
  constexpr int CPS = H2 / NST;       // chunks per score subtile
  static_assert(NPV % 4 == 0 && NSP % 4 == 0 && H2 % NST == 0, "chunks of 4 products");
  constexpr int NSL1 = 10;            // first-half softmax slices

  float mt = kNegInf, msafe = 0.f, alpha = 1.f, psum = 0.f, blk1 = 0.f;
  bool grow = false;
  float blkv[NST][8];
  // First-half slice K: masks and row max (K < 2), exponentials (K >= 2).
  auto slice1 = [&]<int K, bool MASKED>(bool remote, int kb) {
    if constexpr (K < 2) {
      constexpr int s0 = K * ((NST + 1) / 2);
      constexpr int s1 = K ? NST : (NST + 1) / 2;
      if constexpr (MASKED) {
        // key of register r in subtile st is kb + 4*half + (32*st + 8*(r/4) + r%4)
        const int base = kb + 4 * half;
        const int lim = (remote ? rlim : lhi + 1) - base;
        const int lo = remote ? INT32_MIN : llo - base;
#pragma unroll
        for (int st = s0; st < s1; ++st)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int off = 32 * st + 8 * (r >> 2) + (r & 3);
            sc[st][r] = ((off < lim) & (off >= lo)) ? sc[st][r] : kNegInf;
          }
      }
#pragma unroll
      for (int st = s0; st < s1; ++st)
#pragma unroll
        for (int r = 0; r < 16; r += 2) mt = fmaxf(mt, fmaxf(sc[st][r], sc[st][r + 1]));
      if constexpr (K == 1) {
        mt = fmaxf(mt, swap_halves(mt)) * a.scale_log2;
        // lazy rescaling: the max only moves when some row of the wave
        // exceeds it by more than kLazyLog2 (alpha is exactly 1 otherwise)
        const float m = remote ? m_r : m_l;
        grow = __builtin_amdgcn_ballot_w64(mt > m + kLazyLog2) != 0;
        const float mn = grow ? fmaxf(m, mt) : m;
        msafe = mn == kNegInf ? 0.f : mn;
        alpha = fast_exp2(m - msafe);
        if (remote) m_r = mn;
        else m_l = mn;
        mt = kNegInf;
        psum = 0.f;
      }
    } else {
      constexpr int v0 = (16 * NST) * (K - 2) / 8, v1 = (16 * NST) * (K - 1) / 8;
#pragma unroll
      for (int v = v0; v < v1; ++v) {
        const float x = fast_exp2(fmaf(sc[v / 16][v % 16], a.scale_log2, -msafe));
        sc[v / 16][v % 16] = x;
        psum += x;
      }
    }
  };
  // Second-half slice for score subtile ST: the block scaling (remote pass)
  // and the conversion to 16-bit probabilities, after which sc[ST] is free.
  auto slice2 = [&]<int ST>(bool remote) {
    if constexpr (ST == 0) {
      if (remote) zs_r = zs_r * alpha + psum;
      else zs_l = zs_l * alpha + psum;
      if (remote) {
        if constexpr ((1 << LOGB) == NT) {
          // the tile is one block: its row sum is the block sum
          blk1 = psum + swap_halves(psum);
          dr = dr * (alpha * alpha) + psum * blk1;
        } else {
          block_sums<NST, LOGB>(sc, blkv);
          dr *= alpha * alpha;
        }
      }
    }
    if (remote) {
      if constexpr ((1 << LOGB) == NT) {
        sc[ST] *= blk1;
      } else {
        float w = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          sc[ST][r] *= blkv[ST][blk_slot<LOGB>(r)];
          w += sc[ST][r];
        }
        dr += w;
      }
    }
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) pf[ST][c2] = frag_from_c<T>(sc[ST], c2);
  };

  // MASKED = false: an unmasked remote tile (the bulk); MASKED = true: any
  // tile, remote or local, with the causal / window masks applied.
  auto iteration = [&]<int PAR, bool MASKED>(int i) {
    const bool remote = MASKED ? i < n_remote : true;
    wait_vm();
    __syncthreads();
    if (i + 2 < total) kst.template stage<NT>(PAR ? k1s : k0s, tile_of(i + 2) * NT);
    vst.template stage<NT>(PAR ? v1s : v0s, tile_of(i) * NT);
    const T* kt = PAR ? k0s : k1s;
    const T* vt = PAR ? v0s : v1s;
    const int kb = tile_of(i) * NT;
    // chunk g < H1: PV products 4g..4g+3 (head-dim tile q % NDT, 16-key chunk
    // q / NDT); chunk H1 + h: S^T subtile h / CPS, contraction chunks
    // 4 (h % CPS) .. +3
    auto load = [&](int g, int u) -> Frag {
      if (g < H1) {
        const int q = 4 * g + u;
        return vfrag(vt, 16 * (q / NDT), q % NDT);
      }
      const int h = g - H1;
      return kfrag(kt, h / CPS, 4 * (h % CPS) + u);
    };
    Frag buf[2][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) buf[0][u] = load(0, u);
    [&]<int... G>(std::integer_sequence<int, G...>) {
      ([&] {
        constexpr int g = G;
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this chunk's reads
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (g + 1 < H1 + H2) {
#pragma unroll
          for (int u = 0; u < 4; ++u) buf[(g + 1) & 1][u] = load(g + 1, u);
        }
        if constexpr (g < H1) {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int q = 4 * g + u;
            acc[q % NDT] = M::mma(buf[g & 1][u], pf[q / (2 * NDT)][(q / NDT) & 1], acc[q % NDT]);
          }
          [&]<int... L>(std::integer_sequence<int, L...>) {
            (slice1.template operator()<g * NSL1 / H1 + L, MASKED>(remote, kb), ...);
          }(std::make_integer_sequence<int, (g + 1) * NSL1 / H1 - g * NSL1 / H1>{});
        } else {
          constexpr int h = g - H1, st = h / CPS;
          if constexpr (h % CPS == 0) slice2.template operator()<st>(remote);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int c = 4 * (h % CPS) + u;
            sc[st] = M::mma(buf[g & 1][u], qf[c], c == 0 ? zero16() : sc[st]);
          }
        }
      }(), ...);
    }(std::make_integer_sequence<int, H1 + H2>{});
    __builtin_amdgcn_sched_barrier(0);
    // the last remote PV products (tile i-1) are in: park the remote pass;
    // otherwise a raised max rescales the accumulator before the PV products
    // of tile i (next iteration)
    if (i == n_remote) {
      finish_remote();
    } else if (grow) {
      const float f = remote ? alpha * alpha : alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) acc[dt] *= f;
    }
  };

  if (total > 0) {
    // prologue: K of tiles 0 and 1, finite filler in the V buffer iteration 0
    // reads, then the S^T products of tile 0
    kst.template stage<NT>(k0s, tile_of(0) * NT);
    vst.template stage<NT>(v1s, tile_of(0) * NT);
    if (total > 1) kst.template stage<NT>(k1s, tile_of(1) * NT);
    wait_vm();
    __syncthreads();
#pragma unroll
    for (int st = 0; st < NST; ++st) sc[st] = zero16();
    mfma_phase<NST * NKC, 4, 1>([&](int j) { return kfrag(k0s, j / NKC, j % NKC); },
                                [&](int j, Frag f) { sc[j / NKC] = M::mma(f, qf[j % NKC], sc[j / NKC]); });
  }
  // unmasked remote tiles in pairs (an even count; an odd last one joins the
  // masked loop), then every remaining tile through the masked variant
  const int n_fast = max(0, min(full_remote, rs + n_remote) - rs) & ~1;
  int i = 0;
  for (; i < n_fast; i += 2) {
    iteration.template operator()<0, false>(i);
    iteration.template operator()<1, false>(i + 1);
  }
  for (; i < total; i += 2) {
    iteration.template operator()<0, true>(i);
    if (i + 1 < total) iteration.template operator()<1, true>(i + 1);
  }
  if (total > 0) {
    // drain: PV products of the last tile
    wait_vm();
    __syncthreads();
    const T* vt = (total - 1) & 1 ? v1s : v0s;
    mfma_phase<NST * 2 * NDT, 4, 2>(
        [&](int j) { return vfrag(vt, 16 * (j / NDT), j % NDT); },
        [&](int j, Frag f) { acc[j % NDT] = M::mma(f, pf[j / (2 * NDT)][(j / NDT) & 1], acc[j % NDT]); });
  }
  if (total == n_remote) finish_remote();
  // local statistics (zs now holds the local denominator); padding rows,
  // which skipped masks on full remote tiles, have no mass at all
  const float zsum = zs_l + swap_halves(zs_l);
  constexpr int RLD = DP + 4;  // fp32 staging stride: conflict-free 16-byte writes
  static_assert(32 * RLD * 4 + 32 * 4 <= TILE * (int)sizeof(T), "staging fits one buffer");
  float* lst = reinterpret_cast<float*>(wave == 0 ? k0s : (wave == 1 ? k1s : (wave == 2 ? v0s : v1s)));
  // acc * f (per row) into this wave's staging buffer, rows [32 wave, +32)
  auto stage_acc = [&](float f) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 32 * dt + 8 * i + 4 * half;
        const f32x4 lv = {acc[dt][4 * i] * f, acc[dt][4 * i + 1] * f, acc[dt][4 * i + 2] * f,
                          acc[dt][4 * i + 3] * f};
        *reinterpret_cast<f32x4*>(lst + col * RLD + d) = lv;
      }
  };
  if (a.fw0 != nullptr && !piece && threadIdx.x == 0) a.fflag[item] = split ? 1 : 0;
  if (split) {
    // partial results of this piece: statistics per row, and the remote mean
    // (piece 0) or the local mean (piece 1) as rows, for dense_fwd_merge
    const int lrow = wave * 32 + col;
    float* st8 = a.fstat + ((size_t)item * 128 + lrow) * 8;
    if (half == 0 && row_in) {
      if (piece == 0) {
        st8[0] = m_r; st8[1] = zs_r; st8[2] = dr;
      } else {
        st8[3] = m_r; st8[4] = zs_r; st8[5] = dr; st8[6] = m_l; st8[7] = zsum;
      }
    }
    const float f = piece == 0 ? (dr > 0.f ? 1.f / dr : 0.f) : (zsum > 0.f ? 1.f / zsum : 0.f);
    float* dst = (piece == 0 ? a.fw0 : a.fw1) + (size_t)item * 128 * D;
    __syncthreads();  // every wave is done with the K/V buffers
    stage_acc(f);
    __syncthreads();
    constexpr int RL = DP / 4;  // lanes per row, 4 floats each
    const int row0 = qt * 32 * WAVES + wave * 32;
#pragma unroll
    for (int it = 0; it < 32 * RL / 64; ++it) {
      const int r = (it * 64 + lane) / RL, c = ((it * 64 + lane) % RL) * 4;
      if (row0 + r < a.Q)
        *reinterpret_cast<f32x4*>(dst + (int64_t)(wave * 32 + r) * D + c) =
            *reinterpret_cast<const f32x4*>(lst + r * RLD + c);
    }
    return;
  }
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
  const float linv = dl > 0.f ? ploc / dl : 0.f;
  if (half == 0 && row_in) {
    const int64_t sidx = ((int64_t)bi * a.Q + row) * H + hh;
    a.pr[sidx] = prem;
    a.zr[sidx] = log_zr;
    a.z[sidx] = tot;
  }
  // rc = prem * (parked remote mean) and out = rc + ploc * (local mean), in
  // row-contiguous form: each wave stages its 32 rows' local part and weights
  // in one 32 KiB K/V buffer (free after the drain) and then reads, combines
  // and writes whole rows. With lane = row, direct global accesses would
  // touch 64 cache lines per instruction.
  __syncthreads();  // every wave is done with the K/V buffers
  float* wst = lst + 32 * RLD;  // per-row prem
  stage_acc(linv);
  if (half == 0) wst[col] = prem;
  // the parked rc stores of this wave are visible to all its lanes
  __threadfence_block();
  __syncthreads();
  {
    constexpr int RL = DP / 4;  // lanes per row, 4 floats each
    const int row0 = qt * 32 * WAVES + wave * 32;
    typedef T T4 __attribute__((ext_vector_type(4)));
    constexpr int NIT = 32 * RL / 64;
    // every load before the first store (the stores may alias in the
    // compiler's view, which would serialise the round trips)
    f32x4 mean[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int r = (it * 64 + lane) / RL, c = ((it * 64 + lane) % RL) * 4;
      const int64_t g = (((int64_t)bi * a.Q + row0 + r) * H + hh) * D + c;
      mean[it] = row0 + r < a.Q ? *reinterpret_cast<const f32x4*>(a.rc + g) : f32x4{};
    }
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int r = (it * 64 + lane) / RL, c = ((it * 64 + lane) % RL) * 4;
      if (row0 + r < a.Q) {
        const int64_t g = (((int64_t)bi * a.Q + row0 + r) * H + hh) * D + c;
        const float w = wst[r];
        const f32x4 lv = *reinterpret_cast<const f32x4*>(lst + r * RLD + c);
        f32x4 rc;
        T4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          rc[j] = mean[it][j] * w;
          o[j] = from_float<T>(rc[j] + lv[j]);
        }
        *reinterpret_cast<f32x4*>(a.rc + g) = rc;
        *reinterpret_cast<T4*>(reinterpret_cast<T*>(a.out) + g) = o;
      }
    }
  }
}

// Combination of the two pieces of every split row tile: remote partials
// (max m, row sum zs, sum of squared block sums dr, all at scale 2^-m, and
// the remote means) merged at the common max, then the gate with the local
// partial of piece 1 as in the single-piece epilogue. DP/8 threads per row,
// 8 values each: every access is row-contiguous, and all loads of a thread
// are issued before its arithmetic.
template <typename T, int DP>
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
  const float* st8 = a.fstat + ((size_t)item * 128 + lrow) * 8;
  const f32x4 sa = *reinterpret_cast<const f32x4*>(st8), sb = *reinterpret_cast<const f32x4*>(st8 + 4);
  const int64_t p = a.pos[(int64_t)bi * a.Q + row];
  f32x4 mean0[2], mean1[2], meanl[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    mean0[h] = *reinterpret_cast<const f32x4*>(a.fw0 + w + 4 * h);
    mean1[h] = *reinterpret_cast<const f32x4*>(a.rc + g + 4 * h);
    meanl[h] = *reinterpret_cast<const f32x4*>(a.fw1 + w + 4 * h);
  }
  const float m0 = sa[0], zs0 = sa[1], dr0 = sa[2];
  const float m1 = sa[3], zs1 = sb[0], dr1 = sb[1], ml = sb[2], zl = sb[3];
  const float mx = fmaxf(m0, m1);
  float zs = 0.f, w0 = 0.f, w1 = 0.f;
  if (mx != kNegInf) {
    const float e0 = fast_exp2(m0 - mx), e1 = fast_exp2(m1 - mx);
    zs = zs0 * e0 + zs1 * e1;
    w0 = dr0 * e0 * e0;
    w1 = dr1 * e1 * e1;
  }
  const float drs = w0 + w1;
  float log_zr = zs > 0.f ? log_mass(mx, zs) : kNegInf;
  float lr = drs > 0.f ? log_mass(mx, drs) - fast_log2(zs) * kLn2 : kNegInf;
  float ll = zl > 0.f ? log_mass(ml, zl) : kNegInf;
  if (p < 0) { lr = kNegInf; ll = kNegInf; log_zr = kNegInf; }
  const float tot = logaddexp(lr, ll);
  const float safe_total = tot == kNegInf ? 0.f : tot;
  const float prem = lr == kNegInf ? 0.f : __expf(lr - safe_total);
  const float ploc = ll == kNegInf ? 0.f : __expf(ll - safe_total);
  const float a0 = drs > 0.f ? prem * (w0 / drs) : 0.f, a1 = drs > 0.f ? prem * (w1 / drs) : 0.f;
  typedef T T8 __attribute__((ext_vector_type(8)));
  T8 o;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    f32x4 rc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      rc[j] = a0 * mean0[h][j] + a1 * mean1[h][j];
      o[4 * h + j] = from_float<T>(rc[j] + ploc * meanl[h][j]);
    }
    *reinterpret_cast<f32x4*>(a.rc + g + 4 * h) = rc;
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
  // pair mode once slot mode's slots outnumber the compute units
  a.f_pair = a.fw0 != nullptr && 2 * (int64_t)items > device_cus();
  const int per_head = a.f_pair ? 3 * (n_qtiles / 2) + (n_qtiles & 1) : a.fw0 != nullptr ? 2 * n_qtiles : n_qtiles;
  dim3 grid((unsigned)(per_head * a.B * a.H));
  auto go = [&]<int LOGB>() {
    note_launch((const void*)&dense_fwd_fast_kernel<T, DP, LOGB>,
                {"dense_fwd_fast", dtype_code<T>(), DP, 1 << LOGB, 128, 128, 4, 2, grid.x,
                 a.f_pair ? "pair" : (a.fw0 ? "slot" : "grid")});
    hipLaunchKernelGGL((dense_fwd_fast_kernel<T, DP, LOGB>), grid, dim3(256), 0, stream, a, n_qtiles);
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
  note_launch((const void*)&dense_fwd_merge_kernel<T, DP>,
              {"dense_fwd_merge", dtype_code<T>(), DP, a.block, 256 / (DP / 8), DP, 4, 0, items * WPI, "rows"});
  hipLaunchKernelGGL((dense_fwd_merge_kernel<T, DP>), dim3(items * WPI), dim3(256), 0, stream, a, n_qtiles);
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
  const size_t w = align256(items * 128 * (size_t)D * sizeof(float));
  p.off_w1 = w;
  p.off_stat = 2 * w;
  p.off_flag = p.off_stat + align256(items * 128 * 8 * sizeof(float));
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
