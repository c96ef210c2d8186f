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
#include "dense.h"
#include "tile.h"

namespace st {

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
  __shared__ int range[4];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int BH = a.B * a.H;
  const int bh = blockIdx.x % BH;
  const int qt = n_qtiles - 1 - (int)(blockIdx.x / BH);  // longest causal rows first
  const int bi = bh / a.H, hh = bh % a.H;
  const int row = qt * 32 * WAVES + wave * 32 + col;
  const bool row_in = row < a.Q;
  const int64_t H = a.H, D = a.D, N = a.N;
  const int64_t p = row_in ? a.pos[(int64_t)bi * a.Q + row] : -1;
  constexpr int b = 1 << LOGB;

  int rlim = 0, llo = 0, lhi = -1;
  if (p >= 0) {
    const int64_t c = p >> LOGB;
    const int64_t lo = (c - 1) * b > 0 ? (c - 1) * b : 0;
    rlim = (int)(lo < N ? lo : N);
    llo = (int)lo;
    lhi = (int)(p < N - 1 ? p : N - 1);
  }
  if (threadIdx.x == 0) { range[0] = 0; range[1] = 0x7fffffff; range[2] = -1; range[3] = 0x7fffffff; }
  __syncthreads();
  atomicMax(&range[0], rlim);
  if (lhi >= llo) { atomicMin(&range[1], llo); atomicMax(&range[2], lhi); atomicMin(&range[3], rlim); }
  __syncthreads();
  // remote tiles ending at or below every valid row's remote limit need no
  // masks (padding rows are zeroed when the row is finalised)
  const int full_remote = range[3] == 0x7fffffff ? 0 : range[3] / NT;
  const int n_remote = (range[0] + NT - 1) / NT;
  const int lt0 = range[2] >= 0 ? range[1] / NT : 0;
  const int n_local = range[2] >= 0 ? range[2] / NT - lt0 + 1 : 0;
  const int total = n_remote + n_local;
  auto tile_of = [&](int i) { return i < n_remote ? i : lt0 + (i - n_remote); };

  const T* kg = reinterpret_cast<const T*>(a.k) + ((int64_t)bi * N * H + hh) * D;
  const T* vg = reinterpret_cast<const T*>(a.v) + ((int64_t)bi * N * H + hh) * D;
  const int64_t kstride = H * D;
  const Stager<T, DP, WAVES> stager(kstride);
  auto stage = [&]<int BUF>(int i) {
    const int kb = tile_of(i) * NT;
    stager.template stage<NT>(BUF ? k1s : k0s, kg, kstride, kb, a.N);
    stager.template stage<NT>(BUF ? v1s : v0s, vg, kstride, kb, a.N);
  };
  if (total > 0) stage.template operator()<0>(0);

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
  int voff[NDT];
  {
    const int gi = lane >> 4, sl = lane & 15;
    const int r0 = 4 * (gi >> 1) + (sl >> 2);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const int d = 32 * dt + 16 * (gi & 1) + 4 * (sl & 3);
      voff[dt] = r0 * DP + (((d >> 3) ^ swz<DP>(r0)) * 8) + (d & 7);
    }
  }
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef short s8 __attribute__((ext_vector_type(8)));
  auto kfrag = [&](const T* buf, int st, int c) -> Frag {
    return *reinterpret_cast<const Frag*>(buf + 32 * st * DP + koff[c]);
  };
  auto vfrag = [&](const T* buf, int k0, int dt) -> Frag {
    const T* p0 = buf + k0 * DP + voff[dt];
    s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)p0);
    s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)(p0 + 8 * DP));
    return __builtin_bit_cast(Frag, (s8)__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  f32x16 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc[dt] = zero16();
  float m = kNegInf, zs = 0.f, dr = 0.f;
  float log_zr = kNegInf, lr = kNegInf;
  const int64_t obase = (((int64_t)bi * a.Q + row) * H + hh) * D;

  auto finish_remote = [&]() {
    zs += swap_halves(zs);
    dr += swap_halves(dr);
    log_zr = log_mass(m, zs);
    lr = dr > 0.f ? log_mass(m, dr) - fast_log2(zs) * kLn2 : kNegInf;
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
    m = kNegInf;
    zs = 0.f;  // reused as the local denominator
  };

  auto step = [&]<int BUF, bool REMOTE, bool MASKED>(int i) {
    if (i == n_remote) finish_remote();
    const int kb = tile_of(i) * NT;
    wait_vm();
    __syncthreads();
    if (i + 1 < total) stage.template operator()<1 - BUF>(i + 1);
    const T* kt = BUF ? k1s : k0s;
    const T* vt = BUF ? v1s : v0s;

    f32x16 s[NST];
#pragma unroll
    for (int st = 0; st < NST; ++st) s[st] = zero16();
    // product j: subtile j / NKC, contraction chunk j % NKC
    mfma_phase<NST * NKC, 4, 1>([&](int j) { return kfrag(kt, j / NKC, j % NKC); },
                             [&](int j, Frag f) { s[j / NKC] = M::mma(f, qf[j % NKC], s[j / NKC]); });
    // Raw dot products; the scale is applied inside exp2(s*c - m).
    if constexpr (MASKED) {
      // key of register r in subtile st is kb + 4*half + (32*st + 8*(r/4) + r%4):
      // compare the compile-time offset against per-lane thresholds
      const int base = kb + 4 * half;
      const int lim = (REMOTE ? rlim : lhi + 1) - base;
      const int lo = REMOTE ? INT32_MIN : llo - base;
#pragma unroll
      for (int st = 0; st < NST; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          constexpr int dummy = 0;
          const int off = 32 * st + 8 * (r >> 2) + (r & 3) + dummy;
          s[st][r] = ((off < lim) & (off >= lo)) ? s[st][r] : kNegInf;
        }
    }
    float mt = kNegInf;
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int r = 0; r < 16; r += 2) mt = fmaxf(mt, fmaxf(s[st][r], s[st][r + 1]));
    mt = fmaxf(mt, swap_halves(mt)) * a.scale_log2;
    // Lazy rescaling: the running max m only moves when some row's tile max
    // exceeds it by more than kLazyLog2 (so exponents stay below 2^kLazyLog2);
    // otherwise alpha = 1 and the accumulator is left alone.
    float alpha = 1.f;
    if (__builtin_amdgcn_ballot_w64(mt > m + kLazyLog2)) {
      const float mn = fmaxf(m, mt);
      alpha = mn == kNegInf ? 0.f : fast_exp2(m - mn);
      m = mn;
      const float scale_acc = REMOTE ? alpha * alpha : alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) acc[dt] *= scale_acc;
    }
    const float msafe = m == kNegInf ? 0.f : m;
    float psum = 0.f;
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[st][r] = fast_exp2(fmaf(s[st][r], a.scale_log2, -msafe));
        psum += s[st][r];
      }
    zs = zs * alpha + psum;
    if constexpr (REMOTE) {
      float wsum;
      if constexpr ((1 << LOGB) == NT) {
        // the tile is one block: its row sum is the block sum
        const float blk = psum + swap_halves(psum);
#pragma unroll
        for (int st = 0; st < NST; ++st) s[st] *= blk;
        wsum = psum * blk;
      } else {
        float blk[NST][8];
        block_sums<NST, LOGB>(s, blk);
        wsum = 0.f;
#pragma unroll
        for (int st = 0; st < NST; ++st)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            s[st][r] *= blk[st][blk_slot<LOGB>(r)];
            wsum += s[st][r];
          }
      }
      dr = dr * (alpha * alpha) + wsum;
    }
    Frag bp[NST][2];
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) bp[st][c2] = frag_from_c<T>(s[st], c2);
    // product j: 16-key chunk j / NDT, head-dim tile j % NDT
    mfma_phase<NST * 2 * NDT, 4, 2>(
        [&](int j) { return vfrag(vt, 16 * (j / NDT), j % NDT); },
        [&](int j, Frag f) { acc[j % NDT] = M::mma(f, bp[j / (2 * NDT)][(j / NDT) & 1], acc[j % NDT]); });
  };
  auto run = [&]<int BUF>(int i) {
    if (i < n_remote) {
      if (tile_of(i) < full_remote) step.template operator()<BUF, true, false>(i);
      else step.template operator()<BUF, true, true>(i);
    } else {
      step.template operator()<BUF, false, true>(i);
    }
  };
  for (int i = 0; i < total; i += 2) {
    run.template operator()<0>(i);
    if (i + 1 < total) run.template operator()<1>(i + 1);
  }
  if (total == n_remote) finish_remote();
  // local statistics (zs now holds the local denominator); padding rows,
  // which skipped masks on full remote tiles, have no mass at all
  const float zsum = zs + swap_halves(zs);
  const float dl = p >= 0 ? zsum : 0.f;
  const float ll = p >= 0 ? log_mass(m, dl) : kNegInf;
  if (p < 0) {
    lr = kNegInf;
    log_zr = kNegInf;
  }
  const float tot = logaddexp(lr, ll);
  const float safe_total = tot == kNegInf ? 0.f : tot;
  const float prem = lr == kNegInf ? 0.f : __expf(lr - safe_total);
  const float ploc = ll == kNegInf ? 0.f : __expf(ll - safe_total);
  if (!row_in) return;
  const float linv = dl > 0.f ? ploc / dl : 0.f;
  T* og = reinterpret_cast<T*>(a.out);
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = 32 * dt + 8 * i + 4 * half;
      f32x4 rv = *reinterpret_cast<const f32x4*>(a.rc + obase + d);
      f32x4 rc;
      typedef T T4 __attribute__((ext_vector_type(4)));
      T4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        rc[j] = rv[j] * prem;
        o[j] = from_float<T>(rc[j] + acc[dt][4 * i + j] * linv);
      }
      *reinterpret_cast<f32x4*>(a.rc + obase + d) = rc;
      *reinterpret_cast<T4*>(og + obase + d) = o;
    }
  if (half == 0) {
    const int64_t sidx = ((int64_t)bi * a.Q + row) * H + hh;
    a.pr[sidx] = prem;
    a.zr[sidx] = log_zr;
    a.z[sidx] = tot;
  }
}

template <typename T, int DP>
static hipError_t launch_fast(const DenseArgs& a, hipStream_t stream) {
  const int n_qtiles = (a.Q + 127) / 128;
  dim3 grid((unsigned)(n_qtiles * a.B * a.H));
  auto go = [&]<int LOGB>() {
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
  return hipGetLastError();
}

bool dense_fwd_fast_supported(int dtype, const DenseArgs& a) {
  return (dtype == kBF16 || dtype == kF16) && (a.D == 64 || a.D == 128);
}

hipError_t launch_dense_fwd_fast(int dtype, const DenseArgs& a, hipStream_t stream) {
  if (dtype == kBF16) return a.D == 64 ? launch_fast<bf16, 64>(a, stream) : launch_fast<bf16, 128>(a, stream);
  return a.D == 64 ? launch_fast<f16, 64>(a, stream) : launch_fast<f16, 128>(a, stream);
}

}  // namespace st
