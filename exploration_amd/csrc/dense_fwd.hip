// Gated dense block attention, forward (gfx950).
//
// Semantics follow the reference's fused forward
// (st/ops/kernels/dense.py:32-86; st/ops/attention.py:52-93): for a query at
// position p with c = p // b, keys of blocks j < c-1 are remote and take the
// logit a_i + s_j - log Z_R, keys of blocks c-1 and c up to p are local.
//
// Work split: a workgroup owns 32*WAVES query rows of one (batch, head); each
// wave owns 32 rows and computes S^T = K Q^T tiles so that a lane holds one
// row. Key/value tiles of NT keys (whole blocks) are staged in LDS.
//
// Remote pass (one exp per score): with a running row max m,
//   P_i = exp(a_i - m), S_j = sum_{i in j} P_i  (= M_j e^-m),
//   zs = sum_j S_j (= Z_R e^-m), dr = sum_j S_j^2, acc = sum_i P_i S_j v_i,
// so log Z_R = m + log zs, the remote log-mass is m + log dr - log zs and the
// remote mean value is acc / dr. The mean is parked in RC, then a local pass
// (plain online softmax over the window) reuses the accumulator registers.
#include "dense.h"
#include "report.h"
#include "tile.h"

namespace st {

template <typename T, int DP, int NT, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void dense_fwd_kernel(DenseArgs a) {
  typedef Mma<T> M;
  typedef typename M::Frag Frag;
  constexpr int NTHREADS = WAVES * 64;
  constexpr int NST = NT / 32;
  constexpr int NDT = DP / 32;
  constexpr int NKC = DP / M::KW;
  constexpr int LDK = RowLd<T, DP>::value;
  constexpr bool T16 = sizeof(T) == 2;
  constexpr int LDV = T16 ? TLd<NT>::value : RowLd<T, DP>::value;
  constexpr int KBYTES = NT * LDK * (int)sizeof(T);
  constexpr int VBYTES = (T16 ? DP * LDV : NT * LDV) * (int)sizeof(T);
  constexpr bool SHARED = KBYTES + VBYTES > 150 * 1024;  // K then V in one buffer
  __shared__ __attribute__((aligned(16))) T lds_k[SHARED ? (KBYTES > VBYTES ? KBYTES : VBYTES) / sizeof(T)
                                                           : KBYTES / sizeof(T)];
  __shared__ __attribute__((aligned(16))) T lds_v_own[SHARED ? 1 : VBYTES / sizeof(T)];
  T* lds_v = SHARED ? lds_k : lds_v_own;
  __shared__ int range[3][WAVES];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int qt = gridDim.x - 1 - blockIdx.x;  // longest causal rows first
  const int bh = blockIdx.y, bi = bh / a.H, hh = bh % a.H;
  const int row = qt * 32 * WAVES + wave * 32 + col;
  const bool row_in = row < a.Q;
  const int64_t H = a.H, D = a.D, N = a.N;
  const int64_t p = row_in ? a.pos[(int64_t)bi * a.Q + row] : -1;
  const int b = a.block;

  // Per-row key ranges: remote [0, rlim), local [llo, lhi].
  int rlim = 0, llo = 0, lhi = -1;
  if (p >= 0) {
    const int64_t c = p / b;
    const int64_t lo = (c - 1) * b > 0 ? (c - 1) * b : 0;
    rlim = (int)(lo < N ? lo : N);
    llo = (int)lo;
    lhi = (int)(p < N - 1 ? p : N - 1);
  }
  {
    const bool win = lhi >= llo;
    const int r0 = wave_max(rlim), r1 = wave_min(win ? llo : 0x7fffffff), r2 = wave_max(win ? lhi : -1);
    if (lane == 0) { range[0][wave] = r0; range[1][wave] = r1; range[2][wave] = r2; }
  }
  __syncthreads();
  int rg0 = range[0][0], rg1 = range[1][0], rg2 = range[2][0];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) {
    rg0 = max(rg0, range[0][w]);
    rg1 = min(rg1, range[1][w]);
    rg2 = max(rg2, range[2][w]);
  }
  const int n_remote_tiles = (rg0 + NT - 1) / NT;
  const int lt0 = rg2 >= 0 ? rg1 / NT : 0;
  const int lt1 = rg2 >= 0 ? rg2 / NT : -1;

  const T* qg = reinterpret_cast<const T*>(a.q);
  const T* kg = reinterpret_cast<const T*>(a.k) + ((int64_t)bi * N * H + hh) * D;
  const T* vg = reinterpret_cast<const T*>(a.v) + ((int64_t)bi * N * H + hh) * D;
  const int64_t kstride = H * D;

  Frag qf[NKC];
  {
    const T* qrow = qg + (((int64_t)bi * a.Q + (row_in ? row : 0)) * H + hh) * D;
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      const int d = c * M::KW + half * M::VEC;
      if (row_in && d < D) qf[c] = *reinterpret_cast<const Frag*>(qrow + d);
      else qf[c] = Frag{};
    }
  }

  auto stage = [&](int kb, bool keys) {
    if (keys) {
      stage_rows<T, NT, DP, LDK, NTHREADS>(lds_k, kg, kstride, kb, a.N, a.D);
    } else if constexpr (T16) {
      stage_rows_t<T, NT, DP, LDV, NTHREADS>(lds_v, vg, kstride, kb, a.N, a.D);
    } else {
      stage_rows<T, NT, DP, LDV, NTHREADS>(lds_v, vg, kstride, kb, a.N, a.D);
    }
  };

  f32x16 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc[dt] = zero16();
  float m = kNegInf, zs = 0.f, dr = 0.f;

  // ---- remote pass ---------------------------------------------------------
  for (int kt = 0; kt < n_remote_tiles; ++kt) {
    const int kb = kt * NT;
    __syncthreads();
    stage(kb, true);
    if (!SHARED) stage(kb, false);
    __syncthreads();
    f32x16 s[NST];
    scores_t<T, NST, NKC, LDK>(s, lds_k, qf, col, half);
    if (SHARED) { __syncthreads(); stage(kb, false); __syncthreads(); }
    float mt = kNegInf;
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + 32 * st + c_row(r, half);
        const float x = key < rlim ? s[st][r] * a.scale_log2 : kNegInf;
        s[st][r] = x;
        mt = fmaxf(mt, x);
      }
    mt = fmaxf(mt, other_half(mt));
    const float mn = fmaxf(m, mt);
    const float msafe = mn == kNegInf ? 0.f : mn;
    const float alpha = fast_exp2(m - msafe);
    float psum = 0.f;
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int r = 0; r < 16; ++r) { s[st][r] = fast_exp2(s[st][r] - msafe); psum += s[st][r]; }
    zs = zs * alpha + psum;
    dispatch_logb(a.logb, [&]<int LOGB>() {
      float blk[NST][8];
      block_sums<NST, LOGB>(s, blk);
#pragma unroll
      for (int st = 0; st < NST; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[st][r] *= blk[st][blk_slot<LOGB>(r)];
    });
    float wsum = 0.f;
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int r = 0; r < 16; ++r) wsum += s[st][r];
    const float alpha2 = alpha * alpha;
    dr = dr * alpha2 + wsum;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[dt] *= alpha2;
    accumulate_t<T, NST, NDT, LDV>(acc, s, lds_v, col, half);
    m = mn;
  }

  // Remote statistics (both halves of the wave hold the same row values).
  zs += other_half(zs);
  dr += other_half(dr);
  const float log_zr = log_mass(m, zs);
  const float lr = dr > 0.f ? log_mass(m, dr) - fast_log2(zs) * kLn2 : kNegInf;
  const int64_t obase = (((int64_t)bi * a.Q + row) * H + hh) * D;
  {
    const float inv = dr > 0.f ? 1.f / dr : 0.f;
    if (row_in) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 32 * dt + 8 * i + 4 * half;
          if (d < D) {
            f32x4 val = {acc[dt][4 * i] * inv, acc[dt][4 * i + 1] * inv, acc[dt][4 * i + 2] * inv,
                         acc[dt][4 * i + 3] * inv};
            *reinterpret_cast<f32x4*>(a.rc + obase + d) = val;
          }
        }
    }
  }
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc[dt] = zero16();

  // ---- local pass ----------------------------------------------------------
  float ml = kNegInf, dl = 0.f;
  for (int kt = lt0; kt <= lt1; ++kt) {
    const int kb = kt * NT;
    __syncthreads();
    stage(kb, true);
    if (!SHARED) stage(kb, false);
    __syncthreads();
    f32x16 s[NST];
    scores_t<T, NST, NKC, LDK>(s, lds_k, qf, col, half);
    if (SHARED) { __syncthreads(); stage(kb, false); __syncthreads(); }
    float mt = kNegInf;
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + 32 * st + c_row(r, half);
        const float x = (key >= llo && key <= lhi) ? s[st][r] * a.scale_log2 : kNegInf;
        s[st][r] = x;
        mt = fmaxf(mt, x);
      }
    mt = fmaxf(mt, other_half(mt));
    const float mn = fmaxf(ml, mt);
    const float msafe = mn == kNegInf ? 0.f : mn;
    const float alpha = fast_exp2(ml - msafe);
    float psum = 0.f;
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int r = 0; r < 16; ++r) { s[st][r] = fast_exp2(s[st][r] - msafe); psum += s[st][r]; }
    dl = dl * alpha + psum;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[dt] *= alpha;
    accumulate_t<T, NST, NDT, LDV>(acc, s, lds_v, col, half);
    ml = mn;
  }
  dl += other_half(dl);
  const float ll = log_mass(ml, dl);

  // ---- combine -------------------------------------------------------------
  const float total = logaddexp(lr, ll);
  const float safe_total = total == kNegInf ? 0.f : total;
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
      if (d < D) {
        f32x4 rv = *reinterpret_cast<const f32x4*>(a.rc + obase + d);
        f32x4 rc, o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          rc[j] = rv[j] * prem;
          o[j] = rc[j] + acc[dt][4 * i + j] * linv;
        }
        *reinterpret_cast<f32x4*>(a.rc + obase + d) = rc;
#pragma unroll
        for (int j = 0; j < 4; ++j) og[obase + d + j] = from_float<T>(o[j]);
      }
    }
  if (half == 0) {
    const int64_t sidx = ((int64_t)bi * a.Q + row) * H + hh;
    a.pr[sidx] = prem;
    a.zr[sidx] = log_zr;
    a.z[sidx] = total;
  }
}

template <typename T, int DP, int NT>
static hipError_t launch_fwd(const DenseArgs& a, hipStream_t stream) {
  constexpr int WAVES = 4;
  dim3 grid((a.Q + 32 * WAVES - 1) / (32 * WAVES), a.B * a.H);
  note_launch((const void*)&dense_fwd_kernel<T, DP, NT, WAVES>,
              {"dense_fwd", dtype_code<T>(), DP, a.block, 32 * WAVES, NT, WAVES, 1, grid.x * grid.y * grid.z, "grid"});
  hipLaunchKernelGGL((dense_fwd_kernel<T, DP, NT, WAVES>), grid, dim3(WAVES * 64), 0, stream, a);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_fwd_t(const DenseArgs& a, hipStream_t stream) {
  const bool big_block = a.block > 64;
  if (a.D <= 64) return big_block ? launch_fwd<T, 64, 128>(a, stream) : launch_fwd<T, 64, 64>(a, stream);
  if (a.D <= 128) return big_block ? launch_fwd<T, 128, 128>(a, stream) : launch_fwd<T, 128, 64>(a, stream);
  return big_block ? launch_fwd<T, 256, 128>(a, stream) : launch_fwd<T, 256, 64>(a, stream);
}

hipError_t launch_dense_fwd(int dtype, const DenseArgs& a, hipStream_t stream) {
  if (dense_fwd_fast_supported(dtype, a)) return launch_dense_fwd_fast(dtype, a, stream);
  switch (dtype) {
    case kBF16: return launch_fwd_t<bf16>(a, stream);
    case kF16: return launch_fwd_t<f16>(a, stream);
    default: return launch_fwd_t<float>(a, stream);
  }
}

}  // namespace st
