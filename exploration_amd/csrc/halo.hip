// Two-block window attention of the Stack model's local blocks, forward and
// backward (reference st/models/blocks.py:102-179, the attention of
// HaloMemoryBlock.forward_chunk; rotary embedding blocks.py:76-93).
//
// The projection output qkv [B, (G+1)*b, 3, H, hd] is read in place: raw
// block 0 is the previous block (the halo), raw block g+1 the own block of
// query block g. Query block g attends to raw blocks g and g+1 (2b keys),
// key kk visible to query i when kk <= i + b and its absolute position lies
// in [first_key, start + n). Queries are rotated at positions 0..b-1, the
// window keys at -b..b-1, with the caller's cos/sin tables (the reference's
// fp32 angles rounded to the element type); the rotated rows are rounded to
// the element type as the reference's rotary output is.
//
// The work per (block, head) is small (b x 2b scores over hd), so both
// kernels are plain fp32 VALU code on LDS-staged tiles, one wave per unit;
// they are bound by reading qkv once.
//
// Forward: one wave per (batch, query block, head): stage, scores, masked
// softmax, output rows written straight into [B, n, H, hd] (padding rows of
// the last block are not written).
//
// Backward: one wave per (batch, raw block r, head). Block r is the own
// block of query block r-1 and the previous block of query block r; the wave
// recomputes both query blocks' probabilities and writes dq of block r (own
// role) and dk, dv summed over both roles, each role's rotary transposed at
// its own positions. Every row of dqkv has one writer: no atomics, and the
// result does not depend on scheduling. Raw block 0 holds no queries of this
// chunk: its dq is zero.
#include "common.h"
#include "halo.h"
#include "report.h"
#include "tile.h"

namespace st {

namespace {

template <typename T> __device__ __forceinline__ float round_to(float x) { return to_float<T>(from_float<T>(x)); }

template <int B_, int HD>
struct HaloShape {
  static constexpr int HALF = HD / 2, LD = HD + 1, W = 2 * B_, PS = W + 1;
  static constexpr int NP = B_ * HALF / 64;  // (row, j < HALF) pairs per lane
  static constexpr int NE = B_ * HD / 64;    // (row, d) elements per lane
  static_assert(NP >= 1 && B_ * HALF % 64 == 0, "pairs must fill whole waves");
};

// Stage the rotated queries of raw block rq, the rotated window keys of raw
// blocks rk, rk+1 and the window values, as fp32.
template <typename T, int B_, int HD>
__device__ __forceinline__ void stage_window(const HaloArgs& a, const T* qkv, int64_t row0, int h, int rq, int rk,
                                             float* qs, float* ks, float* vs) {
  typedef HaloShape<B_, HD> S;
  const int lane = threadIdx.x;
  const int64_t dim = (int64_t)a.H * HD;
  auto at = [&](int r, int slot, int d) { return ((row0 + r) * 3 + slot) * dim + (int64_t)h * HD + d; };
  for (int e = lane; e < B_ * S::HALF; e += 64) {
    const int i = e / S::HALF, j = e % S::HALF;
    const int r = rq * B_ + i;
    const float lo = to_float<T>(qkv[at(r, 0, j)]), hi = to_float<T>(qkv[at(r, 0, j + S::HALF)]);
    const float c = a.cos_t[(B_ + i) * S::HALF + j], s = a.sin_t[(B_ + i) * S::HALF + j];
    qs[i * S::LD + j] = round_to<T>(lo * c - hi * s);
    qs[i * S::LD + j + S::HALF] = round_to<T>(hi * c + lo * s);
  }
  for (int e = lane; e < S::W * S::HALF; e += 64) {
    const int kk = e / S::HALF, j = e % S::HALF;
    const int r = rk * B_ + kk;
    const float lo = to_float<T>(qkv[at(r, 1, j)]), hi = to_float<T>(qkv[at(r, 1, j + S::HALF)]);
    const float c = a.cos_t[kk * S::HALF + j], s = a.sin_t[kk * S::HALF + j];
    ks[kk * S::LD + j] = round_to<T>(lo * c - hi * s);
    ks[kk * S::LD + j + S::HALF] = round_to<T>(hi * c + lo * s);
  }
  for (int e = lane; e < S::W * HD; e += 64) {
    const int kk = e / HD, d = e % HD;
    vs[kk * S::LD + d] = to_float<T>(qkv[at(rk * B_ + kk, 2, d)]);
  }
}

// Masked scaled scores of query block g, then the row softmax, into ps.
template <int B_, int HD>
__device__ __forceinline__ void window_probs(const HaloArgs& a, int g, const float* qs, const float* ks, float* ps) {
  typedef HaloShape<B_, HD> S;
  const int lane = threadIdx.x;
  for (int e = lane; e < B_ * S::W; e += 64) {
    const int i = e / S::W, kk = e % S::W;
    const int64_t kp = a.start + (int64_t)(g - 1) * B_ + kk;
    const bool ok = kk <= i + B_ && kp >= a.first_key && kp < a.start + a.n;
    float dot = 0.f;
    if (ok) {
#pragma unroll 8
      for (int d = 0; d < HD; ++d) dot += qs[i * S::LD + d] * ks[kk * S::LD + d];
    }
    ps[i * S::PS + kk] = ok ? dot * a.scale : kNegInf;
  }
  __syncthreads();
  for (int i = lane; i < B_; i += 64) {
    float m = kNegInf;
    for (int kk = 0; kk < S::W; ++kk) m = fmaxf(m, ps[i * S::PS + kk]);
    float sum = 0.f;
    for (int kk = 0; kk < S::W; ++kk) {
      const float p = m == kNegInf ? 0.f : __expf(ps[i * S::PS + kk] - m);
      ps[i * S::PS + kk] = p;
      sum += p;
    }
    const float inv = sum > 0.f ? 1.f / sum : 0.f;
    for (int kk = 0; kk < S::W; ++kk) ps[i * S::PS + kk] *= inv;
  }
  __syncthreads();
}

template <typename T, int B_, int HD>
__global__ __launch_bounds__(64) void halo_fwd_kernel(HaloArgs a) {
  typedef HaloShape<B_, HD> S;
  __shared__ float qs[B_ * S::LD], ks[S::W * S::LD], vs[S::W * S::LD], ps[B_ * S::PS];
  const int lane = threadIdx.x;
  const int h = (int)(blockIdx.x % (unsigned)a.H);
  const int g = (int)((blockIdx.x / (unsigned)a.H) % (unsigned)a.G);
  const int bi = (int)(blockIdx.x / ((unsigned)a.H * (unsigned)a.G));
  const int64_t row0 = (int64_t)bi * (a.G + 1) * B_;
  stage_window<T, B_, HD>(a, reinterpret_cast<const T*>(a.qkv), row0, h, g + 1, g, qs, ks, vs);
  __syncthreads();
  window_probs<B_, HD>(a, g, qs, ks, ps);
  T* out = reinterpret_cast<T*>(a.out);
  const int64_t dim = (int64_t)a.H * HD;
  for (int e = lane; e < B_ * HD; e += 64) {
    const int i = e / HD, d = e % HD;
    const int t = g * B_ + i;
    if (t >= a.n) continue;
    float o = 0.f;
#pragma unroll 8
    for (int kk = 0; kk < S::W; ++kk) o += ps[i * S::PS + kk] * vs[kk * S::LD + d];
    out[((int64_t)bi * a.n + t) * dim + (int64_t)h * HD + d] = from_float<T>(o);
  }
}

template <typename T, int B_, int HD>
__global__ __launch_bounds__(64) void halo_bwd_kernel(HaloArgs a) {
  typedef HaloShape<B_, HD> S;
  __shared__ float qs[B_ * S::LD], ks[S::W * S::LD], vs[S::W * S::LD];
  __shared__ float dos[B_ * S::LD], os[B_ * S::LD], ps[B_ * S::PS], dss[B_ * S::PS], delta[B_];
  const int lane = threadIdx.x;
  const int h = (int)(blockIdx.x % (unsigned)a.H);
  const int r = (int)((blockIdx.x / (unsigned)a.H) % (unsigned)(a.G + 1));
  const int bi = (int)(blockIdx.x / ((unsigned)a.H * (unsigned)(a.G + 1)));
  const int64_t row0 = (int64_t)bi * (a.G + 1) * B_;
  const int64_t dim = (int64_t)a.H * HD;
  const T* qkv = reinterpret_cast<const T*>(a.qkv);
  const T* out = reinterpret_cast<const T*>(a.out);
  const T* dout = reinterpret_cast<const T*>(a.dout);
  T* dqkv = reinterpret_cast<T*>(a.dqkv);
  auto at = [&](int row, int slot, int d) { return ((row0 + row) * 3 + slot) * dim + (int64_t)h * HD + d; };

  float dk_lo[S::NP], dk_hi[S::NP], dv[S::NE];
#pragma unroll
  for (int p = 0; p < S::NP; ++p) dk_lo[p] = dk_hi[p] = 0.f;
#pragma unroll
  for (int q = 0; q < S::NE; ++q) dv[q] = 0.f;

  // role 0: block r is the own block of query block r-1 (window rows b..2b-1);
  // role 1: it is the previous block of query block r (window rows 0..b-1)
  for (int role = 0; role < 2; ++role) {
    const int g = role == 0 ? r - 1 : r;
    if (g < 0 || g >= a.G) continue;  // uniform over the wave
    __syncthreads();                   // the previous role's LDS reads are done
    stage_window<T, B_, HD>(a, qkv, row0, h, g + 1, g, qs, ks, vs);
    for (int e = threadIdx.x; e < B_ * HD; e += 64) {
      const int i = e / HD, d = e % HD;
      const int t = g * B_ + i;
      const int64_t o = ((int64_t)bi * a.n + t) * dim + (int64_t)h * HD + d;
      dos[i * S::LD + d] = t < a.n ? to_float<T>(dout[o]) : 0.f;
      os[i * S::LD + d] = t < a.n ? to_float<T>(out[o]) : 0.f;
    }
    __syncthreads();
    for (int i = lane; i < B_; i += 64) {
      float s = 0.f;
      for (int d = 0; d < HD; ++d) s += dos[i * S::LD + d] * os[i * S::LD + d];
      delta[i] = s;
    }
    window_probs<B_, HD>(a, g, qs, ks, ps);  // (its first barrier also publishes delta)
    // dS = P (dP - delta), dP = dO V^T
    for (int e = lane; e < B_ * S::W; e += 64) {
      const int i = e / S::W, kk = e % S::W;
      const float pv = ps[i * S::PS + kk];
      float dp = 0.f;
      if (pv != 0.f) {
#pragma unroll 8
        for (int d = 0; d < HD; ++d) dp += dos[i * S::LD + d] * vs[kk * S::LD + d];
      }
      dss[i * S::PS + kk] = pv * (dp - delta[i]);
    }
    __syncthreads();
    if (role == 0) {
      // dq of block r = scale * dS K, rotary transposed at query positions
      for (int e = lane; e < B_ * S::HALF; e += 64) {
        const int i = e / S::HALF, j = e % S::HALF;
        float lo = 0.f, hi = 0.f;
        for (int kk = 0; kk < S::W; ++kk) {
          const float ds = dss[i * S::PS + kk];
          lo += ds * ks[kk * S::LD + j];
          hi += ds * ks[kk * S::LD + j + S::HALF];
        }
        lo *= a.scale;
        hi *= a.scale;
        const float c = a.cos_t[(B_ + i) * S::HALF + j], s = a.sin_t[(B_ + i) * S::HALF + j];
        dqkv[at(r * B_ + i, 0, j)] = from_float<T>(lo * c + hi * s);
        dqkv[at(r * B_ + i, 0, j + S::HALF)] = from_float<T>(hi * c - lo * s);
      }
    }
    // this role's dk (scale * dS^T Q, rotary transposed at the window
    // positions of block r) and dv (P^T dO)
    const int kk0 = role == 0 ? B_ : 0;
#pragma unroll
    for (int p = 0; p < S::NP; ++p) {
      const int e = lane + 64 * p;
      const int i2 = e / S::HALF, j = e % S::HALF, kk = kk0 + i2;
      float lo = 0.f, hi = 0.f;
      for (int i = 0; i < B_; ++i) {
        const float ds = dss[i * S::PS + kk];
        lo += ds * qs[i * S::LD + j];
        hi += ds * qs[i * S::LD + j + S::HALF];
      }
      lo *= a.scale;
      hi *= a.scale;
      const float c = a.cos_t[kk * S::HALF + j], s = a.sin_t[kk * S::HALF + j];
      dk_lo[p] += lo * c + hi * s;
      dk_hi[p] += hi * c - lo * s;
    }
#pragma unroll
    for (int q = 0; q < S::NE; ++q) {
      const int e = lane + 64 * q;
      const int i2 = e / HD, d = e % HD, kk = kk0 + i2;
      float acc = 0.f;
      for (int i = 0; i < B_; ++i) acc += ps[i * S::PS + kk] * dos[i * S::LD + d];
      dv[q] += acc;
    }
  }
  if (r == 0) {
    for (int e = lane; e < B_ * HD; e += 64) dqkv[at(e / HD, 0, e % HD)] = from_float<T>(0.f);
  }
#pragma unroll
  for (int p = 0; p < S::NP; ++p) {
    const int e = lane + 64 * p;
    const int i2 = e / S::HALF, j = e % S::HALF;
    dqkv[at(r * B_ + i2, 1, j)] = from_float<T>(dk_lo[p]);
    dqkv[at(r * B_ + i2, 1, j + S::HALF)] = from_float<T>(dk_hi[p]);
  }
#pragma unroll
  for (int q = 0; q < S::NE; ++q) {
    const int e = lane + 64 * q;
    dqkv[at(r * B_ + e / HD, 2, e % HD)] = from_float<T>(dv[q]);
  }
}

// ---------------------------------------------------------------------------
// head_dim 64 (the stack_100m shape): register-blocked variants. The loops
// above load both operands of every FMA from LDS; these keep one operand in
// registers and read the other as 16-byte broadcasts.
//  * row phases (scores, dP): lane = key kk + W * slice; the lane holds its
//    key's K (and V) slice of 64 / LPK dims, every query (dO) row is a
//    broadcast read, the LPK slice sums meet through cross-lane adds;
//  * column phases (output, dq, dk, dv): lane = head-dim column d; the lane
//    holds its column of V, K, Q or dO, the P / dS rows are broadcast reads,
//    and the rotary transposes of dq and dk pair column d with lane d ^ 32.
// The staged tiles keep the element type (the rotated rows are rounded to
// it anyway): half the LDS of fp32 tiles, so more one-wave workgroups share
// a CU and hide each other's memory waits.
template <typename T, int B_>
struct Halo64 {
  static constexpr int HD = 64, HALF = 32, W = 2 * B_, LPK = 64 / W, SL = HD / LPK;
  static constexpr int E = Vec16<T>::n;          // elements per 16-byte read
  static constexpr int LD = HD + E;              // element-type rows, 16-byte aligned
  static constexpr int PS = W + 4;               // fp32 probability rows
  static_assert(LPK >= 1 && SL % E == 0 && W % 4 == 0, "shape");
};

// Stage query block g (rotated), its window keys (rotated) and values in the
// element type. Every global load of the unit is issued before the first
// store (16-byte vectors, clamped indices instead of predicates), so the
// wave waits for one memory round trip, not one per element.
template <typename T, int B_>
__device__ __forceinline__ void stage64(const HaloArgs& a, const T* qkv, int64_t row0, int h, int g, T* qs, T* ks,
                                        T* vs) {
  typedef Halo64<T, B_> S;
  typedef typename Vec16<T>::type V;
  constexpr int E = S::E, VPR = S::HD / E, HV = VPR / 2, E4 = E / 4;
  constexpr int NQ = B_ * HV, NK = S::W * HV, NV = S::W * VPR;
  constexpr int TQ = (NQ + 63) / 64, TK = (NK + 63) / 64, TV = (NV + 63) / 64;
  const int lane = threadIdx.x;
  const int64_t dim = (int64_t)a.H * S::HD;
  auto src = [&](int r, int slot, int d) { return qkv + ((row0 + r) * 3 + slot) * dim + (int64_t)h * S::HD + d; };
  V ql[TQ], qh[TQ], kl[TK], kh[TK], vv[TV];
  f32x4 qc[TQ][E4], qn[TQ][E4], kc[TK][E4], kn[TK][E4];
#pragma unroll
  for (int t = 0; t < TQ; ++t) {
    const int e = min(lane + 64 * t, NQ - 1), i = e / HV, c = e % HV;
    ql[t] = load_vec<V>(src((g + 1) * B_ + i, 0, c * E));
    qh[t] = load_vec<V>(src((g + 1) * B_ + i, 0, c * E + S::HALF));
#pragma unroll
    for (int u = 0; u < E4; ++u) {
      qc[t][u] = load_vec<f32x4>(a.cos_t + (B_ + i) * S::HALF + c * E + 4 * u);
      qn[t][u] = load_vec<f32x4>(a.sin_t + (B_ + i) * S::HALF + c * E + 4 * u);
    }
  }
#pragma unroll
  for (int t = 0; t < TK; ++t) {
    const int e = min(lane + 64 * t, NK - 1), kk = e / HV, c = e % HV;
    kl[t] = load_vec<V>(src(g * B_ + kk, 1, c * E));
    kh[t] = load_vec<V>(src(g * B_ + kk, 1, c * E + S::HALF));
#pragma unroll
    for (int u = 0; u < E4; ++u) {
      kc[t][u] = load_vec<f32x4>(a.cos_t + kk * S::HALF + c * E + 4 * u);
      kn[t][u] = load_vec<f32x4>(a.sin_t + kk * S::HALF + c * E + 4 * u);
    }
  }
#pragma unroll
  for (int t = 0; t < TV; ++t) {
    const int e = min(lane + 64 * t, NV - 1), kk = e / VPR, c = e % VPR;
    vv[t] = load_vec<V>(src(g * B_ + kk, 2, c * E));
  }
#pragma unroll
  for (int t = 0; t < TQ; ++t) {
    const int e = lane + 64 * t, i = min(e, NQ - 1) / HV, c = e % HV;
    if (e >= NQ) break;
    V lo_out, hi_out;
#pragma unroll
    for (int u = 0; u < E; ++u) {
      const float lo = to_float<T>(ql[t][u]), hi = to_float<T>(qh[t][u]);
      const float cs = qc[t][u / 4][u % 4], sn = qn[t][u / 4][u % 4];
      lo_out[u] = from_float<T>(lo * cs - hi * sn);
      hi_out[u] = from_float<T>(hi * cs + lo * sn);
    }
    *reinterpret_cast<V*>(qs + i * S::LD + c * E) = lo_out;
    *reinterpret_cast<V*>(qs + i * S::LD + c * E + S::HALF) = hi_out;
  }
#pragma unroll
  for (int t = 0; t < TK; ++t) {
    const int e = lane + 64 * t, kk = min(e, NK - 1) / HV, c = e % HV;
    if (e >= NK) break;
    V lo_out, hi_out;
#pragma unroll
    for (int u = 0; u < E; ++u) {
      const float lo = to_float<T>(kl[t][u]), hi = to_float<T>(kh[t][u]);
      const float cs = kc[t][u / 4][u % 4], sn = kn[t][u / 4][u % 4];
      lo_out[u] = from_float<T>(lo * cs - hi * sn);
      hi_out[u] = from_float<T>(hi * cs + lo * sn);
    }
    *reinterpret_cast<V*>(ks + kk * S::LD + c * E) = lo_out;
    *reinterpret_cast<V*>(ks + kk * S::LD + c * E + S::HALF) = hi_out;
  }
#pragma unroll
  for (int t = 0; t < TV; ++t) {
    const int e = lane + 64 * t, kk = min(e, NV - 1) / VPR, c = e % VPR;
    if (e >= NV) break;
    *reinterpret_cast<V*>(vs + kk * S::LD + c * E) = vv[t];
  }
}

// dO rows of query block g in the element type (zero beyond the n real rows)
// and delta = rowsum(dO * O) from the same loads (the VPR lanes of a row
// reduce through cross-lane adds): O itself is never staged.
template <typename T, int B_>
__device__ __forceinline__ void stage_rows64(const HaloArgs& a, int bi, int h, int g, T* dos, float* delta) {
  typedef Halo64<T, B_> S;
  typedef typename Vec16<T>::type V;
  constexpr int E = S::E, VPR = S::HD / E, N = B_ * VPR, TT = (N + 63) / 64;
  const int lane = threadIdx.x;
  const int64_t dim = (int64_t)a.H * S::HD;
  const T* dout = reinterpret_cast<const T*>(a.dout);
  const T* out = reinterpret_cast<const T*>(a.out);
  V gv[TT], ov[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int e = min(lane + 64 * t, N - 1), i = e / VPR, c = e % VPR;
    const int row = min(g * B_ + i, a.n - 1);
    const int64_t o = ((int64_t)bi * a.n + row) * dim + (int64_t)h * S::HD + c * E;
    gv[t] = load_vec<V>(dout + o);
    ov[t] = load_vec<V>(out + o);
  }
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int e = lane + 64 * t, i = min(e, N - 1) / VPR, c = e % VPR;
    const bool real = g * B_ + i < a.n;
    float sd = 0.f;
#pragma unroll
    for (int u = 0; u < E; ++u) sd += to_float<T>(gv[t][u]) * to_float<T>(ov[t][u]);
#pragma unroll
    for (int off = 1; off < VPR; off <<= 1) sd += __shfl_xor(sd, off, 64);  // every lane takes part
    if (e < N) {  // N is a multiple of VPR: a row's lanes agree
      if (!real) {
        sd = 0.f;
#pragma unroll
        for (int u = 0; u < E; ++u) gv[t][u] = from_float<T>(0.f);
      }
      *reinterpret_cast<V*>(dos + i * S::LD + c * E) = gv[t];
      if (c == 0) delta[i] = sd;
    }
  }
}

// Sum over the LPK lanes holding slices of one key (lanes kk + W * slice).
template <int W>
__device__ __forceinline__ float slice_sum(float x) {
#pragma unroll
  for (int off = W; off < 64; off <<= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// Dot of an element-type LDS row slice (broadcast reads) with fp32 registers.
template <typename T, int N>
__device__ __forceinline__ float dot_row(const T* row, const float (&reg)[N]) {
  typedef typename Vec16<T>::type V;
  constexpr int E = Vec16<T>::n;
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < N; c += E) {
    const V v = *reinterpret_cast<const V*>(row + c);
#pragma unroll
    for (int u = 0; u < E; ++u) s += to_float<T>(v[u]) * reg[c + u];
  }
  return s;
}

// Dot of an fp32 LDS row (broadcast reads) with fp32 registers.
template <int N>
__device__ __forceinline__ float dot_bcast(const float* row, const float (&reg)[N]) {
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < N; c += 4) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(row + c);
    s += v[0] * reg[c] + v[1] * reg[c + 1] + v[2] * reg[c + 2] + v[3] * reg[c + 3];
  }
  return s;
}

// Masked scores of query block g (row phase) and their row softmax, into ps.
template <typename T, int B_>
__device__ __forceinline__ void probs64(const HaloArgs& a, int g, const T* qs,
                                        const float (&kreg)[Halo64<T, B_>::SL], float* ps) {
  typedef Halo64<T, B_> S;
  const int lane = threadIdx.x, kk = lane % S::W, sl = lane / S::W;
  const int64_t kp = a.start + (int64_t)(g - 1) * B_ + kk;
  const bool key_ok = kp >= a.first_key && kp < a.start + a.n;
#pragma unroll 4
  for (int i = 0; i < B_; ++i) {
    const float s = slice_sum<S::W>(dot_row<T>(qs + i * S::LD + sl * S::SL, kreg));
    if (sl == 0) ps[i * S::PS + kk] = (key_ok && kk <= i + B_) ? s * a.scale : kNegInf;
  }
  __syncthreads();
  // row softmax, LPR adjacent lanes per row (each holds W / LPR scores)
  constexpr int LPR = 64 / B_ < S::W ? 64 / B_ : S::W, PER = S::W / LPR;
  if (lane < B_ * LPR) {
    const int i = lane / LPR, part = lane % LPR;
    float v[PER];
    float m = kNegInf;
#pragma unroll
    for (int t = 0; t < PER; ++t) {
      v[t] = ps[i * S::PS + part + LPR * t];
      m = fmaxf(m, v[t]);
    }
#pragma unroll
    for (int off = 1; off < LPR; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    float sum = 0.f;
#pragma unroll
    for (int t = 0; t < PER; ++t) {
      v[t] = m == kNegInf ? 0.f : __expf(v[t] - m);
      sum += v[t];
    }
#pragma unroll
    for (int off = 1; off < LPR; off <<= 1) sum += __shfl_xor(sum, off, 64);
    const float inv = sum > 0.f ? 1.f / sum : 0.f;
#pragma unroll
    for (int t = 0; t < PER; ++t) ps[i * S::PS + part + LPR * t] = v[t] * inv;
  }
  __syncthreads();
}

// The rotary transpose of a gradient column held as lane = d: the partner
// column d ^ 32 comes from the lane d ^ 32.
__device__ __forceinline__ float rotary_back(float dy, int d, const float* cos_row, const float* sin_row) {
  const float other = __shfl_xor(dy, 32, 64);
  const float c = cos_row[d & 31], s = sin_row[d & 31];
  return d < 32 ? dy * c + other * s : dy * c - other * s;
}

template <typename T, int B_>
__global__ __launch_bounds__(64) void halo_fwd64_kernel(HaloArgs a) {
  typedef Halo64<T, B_> S;
  __shared__ __attribute__((aligned(16))) T qs[B_ * S::LD], ks[S::W * S::LD], vs[S::W * S::LD];
  __shared__ __attribute__((aligned(16))) float ps[B_ * S::PS];
  const int lane = threadIdx.x;
  const int h = (int)(blockIdx.x % (unsigned)a.H);
  const int g = (int)((blockIdx.x / (unsigned)a.H) % (unsigned)a.G);
  const int bi = (int)(blockIdx.x / ((unsigned)a.H * (unsigned)a.G));
  const int64_t row0 = (int64_t)bi * (a.G + 1) * B_;
  stage64<T, B_>(a, reinterpret_cast<const T*>(a.qkv), row0, h, g, qs, ks, vs);
  __syncthreads();
  float kreg[S::SL];
  {
    const int kk = lane % S::W, sl = lane / S::W;
#pragma unroll
    for (int c = 0; c < S::SL; ++c) kreg[c] = to_float<T>(ks[kk * S::LD + sl * S::SL + c]);
  }
  probs64<T, B_>(a, g, qs, kreg, ps);
  float vcol[S::W];
#pragma unroll
  for (int kk = 0; kk < S::W; ++kk) vcol[kk] = to_float<T>(vs[kk * S::LD + lane]);
  T* out = reinterpret_cast<T*>(a.out);
  const int64_t dim = (int64_t)a.H * S::HD;
#pragma unroll 4
  for (int i = 0; i < B_; ++i) {
    const int t = g * B_ + i;
    if (t >= a.n) break;
    out[((int64_t)bi * a.n + t) * dim + (int64_t)h * S::HD + lane] = from_float<T>(dot_bcast(ps + i * S::PS, vcol));
  }
}

template <typename T, int B_>
__global__ __launch_bounds__(64) void halo_bwd64_kernel(HaloArgs a) {
  typedef Halo64<T, B_> S;
  __shared__ __attribute__((aligned(16))) T qs[B_ * S::LD], ks[S::W * S::LD], vs[S::W * S::LD];
  __shared__ __attribute__((aligned(16))) T dos[B_ * S::LD];
  __shared__ __attribute__((aligned(16))) float ps[B_ * S::PS], dss[B_ * S::PS];
  __shared__ float delta[B_];
  const int lane = threadIdx.x;
  const int h = (int)(blockIdx.x % (unsigned)a.H);
  const int r = (int)((blockIdx.x / (unsigned)a.H) % (unsigned)(a.G + 1));
  const int bi = (int)(blockIdx.x / ((unsigned)a.H * (unsigned)(a.G + 1)));
  const int64_t row0 = (int64_t)bi * (a.G + 1) * B_;
  const int64_t dim = (int64_t)a.H * S::HD;
  const T* qkv = reinterpret_cast<const T*>(a.qkv);
  T* dqkv = reinterpret_cast<T*>(a.dqkv);
  auto at = [&](int row, int slot, int d) { return ((row0 + row) * 3 + slot) * dim + (int64_t)h * S::HD + d; };
  const int kk_l = lane % S::W, sl = lane / S::W, d = lane;

  // column d of dk and dv of block r's rows, summed over both roles
  float dk[B_], dv[B_];
#pragma unroll
  for (int i = 0; i < B_; ++i) dk[i] = dv[i] = 0.f;

  for (int role = 0; role < 2; ++role) {
    const int g = role == 0 ? r - 1 : r;  // role 0: own block of query block r-1; role 1: previous of query block r
    if (g < 0 || g >= a.G) continue;      // uniform over the wave
    __syncthreads();
    stage64<T, B_>(a, qkv, row0, h, g, qs, ks, vs);
    stage_rows64<T, B_>(a, bi, h, g, dos, delta);
    __syncthreads();
    {
      float kreg[S::SL];
#pragma unroll
      for (int c = 0; c < S::SL; ++c) kreg[c] = to_float<T>(ks[kk_l * S::LD + sl * S::SL + c]);
      probs64<T, B_>(a, g, qs, kreg, ps);
    }
    float vreg[S::SL];
#pragma unroll
    for (int c = 0; c < S::SL; ++c) vreg[c] = to_float<T>(vs[kk_l * S::LD + sl * S::SL + c]);
    // dS = P (dP - delta) with dP = dO V^T (row phase)
#pragma unroll 2
    for (int i = 0; i < B_; ++i) {
      const float dp = slice_sum<S::W>(dot_row<T>(dos + i * S::LD + sl * S::SL, vreg));
      if (sl == 0) dss[i * S::PS + kk_l] = ps[i * S::PS + kk_l] * (dp - delta[i]);
    }
    __syncthreads();
    // column phase, lane = d
    if (role == 0) {
      // dq of block r = scale * dS K, transposed through the query rotary
      float kcol[S::W];
#pragma unroll
      for (int kk = 0; kk < S::W; ++kk) kcol[kk] = to_float<T>(ks[kk * S::LD + d]);
#pragma unroll 4
      for (int i = 0; i < B_; ++i) {
        const float dy = a.scale * dot_bcast(dss + i * S::PS, kcol);
        const float dx = rotary_back(dy, d, a.cos_t + (B_ + i) * S::HALF, a.sin_t + (B_ + i) * S::HALF);
        dqkv[at(r * B_ + i, 0, d)] = from_float<T>(dx);
      }
    }
    // this role's window rows kk0 + i2 are block r's rows i2; dv and the
    // unrotated dk take P / dS rows as 16-byte broadcasts
    const int kk0 = role == 0 ? B_ : 0;
    float sk[B_];
#pragma unroll
    for (int i2 = 0; i2 < B_; ++i2) sk[i2] = 0.f;
#pragma unroll 2
    for (int i = 0; i < B_; ++i) {
      const float qv = to_float<T>(qs[i * S::LD + d]), gv = to_float<T>(dos[i * S::LD + d]);
#pragma unroll
      for (int i2 = 0; i2 < B_; i2 += 4) {
        const f32x4 p4 = *reinterpret_cast<const f32x4*>(ps + i * S::PS + kk0 + i2);
        const f32x4 s4 = *reinterpret_cast<const f32x4*>(dss + i * S::PS + kk0 + i2);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          dv[i2 + u] += p4[u] * gv;
          sk[i2 + u] += s4[u] * qv;
        }
      }
    }
#pragma unroll
    for (int i2 = 0; i2 < B_; ++i2)
      dk[i2] += rotary_back(a.scale * sk[i2], d, a.cos_t + (kk0 + i2) * S::HALF, a.sin_t + (kk0 + i2) * S::HALF);
  }
  if (r == 0) {
#pragma unroll
    for (int i = 0; i < B_; ++i) dqkv[at(i, 0, d)] = from_float<T>(0.f);
  }
#pragma unroll
  for (int i2 = 0; i2 < B_; ++i2) {
    dqkv[at(r * B_ + i2, 1, d)] = from_float<T>(dk[i2]);
    dqkv[at(r * B_ + i2, 2, d)] = from_float<T>(dv[i2]);
  }
}

// ---------------------------------------------------------------------------
// b = 16, head_dim 64, 16-bit elements: the five products on MFMA
// (v_mfma_f32_16x16x32: lane l holds A[l%16][8(l/16)+s], B[8(l/16)+s][l%16]
// and C[4(l/16)+r][l%16]). Scores are computed transposed, S^T = K Q^T, so
// lane l owns query row l%16 and keys 16t + 4(l/16) + r (t = 0, 1; r = 0..3):
// row reductions are in-lane plus two exchanges (lanes l ^ 16, l ^ 32). The
// same registers, packed in that key order, are the A operand of P V and
// dS K; their B operand reads V and K from transposed LDS copies in the same
// permuted key order (slot 8(l/16)+s holds key 4(l/16)+s for s < 4 and
// 16+4(l/16)+s-4 for s >= 4). dK and dV contract over the block's 16 query
// rows: the k slots 16..31 (lanes 32..63) are zero.
struct HaloMfma {
  static constexpr int B_ = 16, W = 32, HD = 64, HALF = 32;
  static constexpr int LD = HD + 8;  // row-major 16-bit tiles (144-byte rows)
  static constexpr int LR = B_ + 8;  // P^T, dS^T: [key][row]
};

template <typename T>
using Vec4 = T __attribute__((ext_vector_type(4)));

// The global loads of one unit (query block g of batch row bi, head h): the
// query block, its window keys and values, their rotary cos/sin, and for the
// backward the block's dO and O rows. Loading and storing are separate so
// the backward can have the next unit's loads in flight during the products.
template <typename T>
struct HaloLoads {
  typedef typename Vec16<T>::type V;
  V ql, qh, kl[2], kh[2], vv[4], gv[2], ov[2];
  f32x4 qcs[2], qsn[2], kcs[2][2], ksn[2][2];
};

// PARTS selects what to load / store: bit 0 the query block and window keys
// (with their cos/sin), bit 1 the values and, for the backward, dO and O.
template <typename T, bool BWD, int PARTS = 3>
__device__ __forceinline__ void load_unit(const HaloArgs& a, int64_t row0, int bi, int h, int g, HaloLoads<T>& L) {
  typedef HaloMfma S;
  typedef typename Vec16<T>::type V;
  constexpr int E = 8, VPR = S::HD / E, HV = VPR / 2;
  const int lane = threadIdx.x;
  const int64_t dim = (int64_t)a.H * S::HD;
  const T* qkv = reinterpret_cast<const T*>(a.qkv);
  auto src = [&](int r, int slot, int d) { return qkv + ((row0 + r) * 3 + slot) * dim + (int64_t)h * S::HD + d; };
  const int qi = lane / HV, qc = lane % HV;
  if constexpr (PARTS & 1) {
  L.ql = load_vec<V>(src((g + 1) * S::B_ + qi, 0, qc * E));
  L.qh = load_vec<V>(src((g + 1) * S::B_ + qi, 0, qc * E + S::HALF));
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    L.qcs[u] = load_vec<f32x4>(a.cos_t + (S::B_ + qi) * S::HALF + qc * E + 4 * u);
    L.qsn[u] = load_vec<f32x4>(a.sin_t + (S::B_ + qi) * S::HALF + qc * E + 4 * u);
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int e = lane + 64 * t, kk = e / HV, c = e % HV;
    L.kl[t] = load_vec<V>(src(g * S::B_ + kk, 1, c * E));
    L.kh[t] = load_vec<V>(src(g * S::B_ + kk, 1, c * E + S::HALF));
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      L.kcs[t][u] = load_vec<f32x4>(a.cos_t + kk * S::HALF + c * E + 4 * u);
      L.ksn[t][u] = load_vec<f32x4>(a.sin_t + kk * S::HALF + c * E + 4 * u);
    }
  }
  }
  if constexpr ((PARTS & 2) != 0) {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int e = lane + 64 * t, kk = e / VPR, c = e % VPR;
    L.vv[t] = load_vec<V>(src(g * S::B_ + kk, 2, c * E));
  }
  }
  if (BWD && (PARTS & 2)) {
    const T* dout = reinterpret_cast<const T*>(a.dout);
    const T* out = reinterpret_cast<const T*>(a.out);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int e = lane + 64 * t, i = e / VPR, c = e % VPR;
      const int row = min(g * S::B_ + i, a.n - 1);
      const int64_t o = ((int64_t)bi * a.n + row) * dim + (int64_t)h * S::HD + c * E;
      L.gv[t] = load_vec<V>(dout + o);
      L.ov[t] = load_vec<V>(out + o);
    }
  }
}

// Store a unit's loads as row-major tiles: the query block and its window
// keys rotated, the values, and for the backward dO (zero beyond the n real
// rows) and delta = rowsum(dO * O). Operands that need the transpose read
// these tiles with ds_read_tr16_b64 (frag_tr_rows).
template <typename T, bool BWD, int PARTS = 3>
__device__ __forceinline__ void store_unit(const HaloArgs& a, const HaloLoads<T>& L, int g, T* qs, T* ks, T* vs,
                                           T* dos, float* delta) {
  typedef HaloMfma S;
  typedef typename Vec16<T>::type V;
  constexpr int E = 8, VPR = S::HD / E, HV = VPR / 2;
  const int lane = threadIdx.x;
  // rotate a (lo, hi) pair of 8-element chunks of one row
  auto put = [&](const V& lo, const V& hi, const f32x4 (&cs)[2], const f32x4 (&sn)[2], int row, int c, T* rows) {
    V lo_out, hi_out;
#pragma unroll
    for (int u = 0; u < E; ++u) {
      const float x = to_float<T>(lo[u]), y = to_float<T>(hi[u]);
      const float cu = cs[u / 4][u % 4], su = sn[u / 4][u % 4];
      lo_out[u] = from_float<T>(x * cu - y * su);
      hi_out[u] = from_float<T>(y * cu + x * su);
    }
    *reinterpret_cast<V*>(rows + row * S::LD + c * E) = lo_out;
    *reinterpret_cast<V*>(rows + row * S::LD + c * E + S::HALF) = hi_out;
  };
  if constexpr (PARTS & 1) {
    put(L.ql, L.qh, L.qcs, L.qsn, lane / HV, lane % HV, qs);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int e = lane + 64 * t;
      put(L.kl[t], L.kh[t], L.kcs[t], L.ksn[t], e / HV, e % HV, ks);
    }
  }
  if constexpr ((PARTS & 2) != 0) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int e = lane + 64 * t, kk = e / VPR, c = e % VPR;
      *reinterpret_cast<V*>(vs + kk * S::LD + c * E) = L.vv[t];
    }
  }
  if (BWD && (PARTS & 2)) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int e = lane + 64 * t, i = e / VPR, c = e % VPR;
      float sd = 0.f;
#pragma unroll
      for (int u = 0; u < E; ++u) sd += to_float<T>(L.gv[t][u]) * to_float<T>(L.ov[t][u]);
#pragma unroll
      for (int off = 1; off < VPR; off <<= 1) sd += __shfl_xor(sd, off, 64);
      V gz = L.gv[t];
      if (g * S::B_ + i >= a.n) {
        sd = 0.f;
#pragma unroll
        for (int u = 0; u < E; ++u) gz[u] = from_float<T>(0.f);
      }
      *reinterpret_cast<V*>(dos + i * S::LD + c * E) = gz;
      if (c == 0) delta[i] = sd;
    }
  }
}

// Transposed score-shaped tiles: c[t][r] = sum_d A[16t + 4(l/16) + r][d] * B[l%16][d]
// with A = the row-major window tile (keys) and B the row-major query-block
// tile: S^T from (K, Q), dP^T from (V, dO).
template <typename T>
__device__ __forceinline__ void window_tiles(const T* as, const T* bs, f32x4 (&c)[2]) {
  typedef HaloMfma S;
  typedef Mma16<T> M;
  typedef typename M::Frag F;
  const int lane = threadIdx.x, col = lane & 15, grp = lane >> 4;
  const F b0 = *reinterpret_cast<const F*>(bs + col * S::LD + 8 * grp);
  const F b1 = *reinterpret_cast<const F*>(bs + col * S::LD + 32 + 8 * grp);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const F a0 = *reinterpret_cast<const F*>(as + (16 * t + col) * S::LD + 8 * grp);
    const F a1 = *reinterpret_cast<const F*>(as + (16 * t + col) * S::LD + 32 + 8 * grp);
    c[t] = M::mma(a1, b1, M::mma(a0, b0, f32x4{0.f, 0.f, 0.f, 0.f}));
  }
}

// Mask, scale and softmax of query row l%16 of block g; s holds S^T tiles in,
// probabilities out.
__device__ __forceinline__ void window_softmax(const HaloArgs& a, int g, f32x4 (&s)[2]) {
  typedef HaloMfma S;
  const int lane = threadIdx.x, i = lane & 15, grp = lane >> 4;
  float m = kNegInf;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kk = 16 * t + 4 * grp + r;
      const int64_t kp = a.start + (int64_t)(g - 1) * S::B_ + kk;
      const bool ok = kp >= a.first_key && kp < a.start + a.n && kk <= i + S::B_;
      s[t][r] = ok ? s[t][r] * a.scale : kNegInf;
      m = fmaxf(m, s[t][r]);
    }
  }
  m = fmaxf(m, __shfl_xor(m, 16, 64));
  m = fmaxf(m, __shfl_xor(m, 32, 64));
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s[t][r] = m == kNegInf ? 0.f : __expf(s[t][r] - m);
      sum += s[t][r];
    }
  }
  sum += __shfl_xor(sum, 16, 64);
  sum += __shfl_xor(sum, 32, 64);
  const float inv = sum > 0.f ? 1.f / sum : 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t) s[t] *= inv;
}

// A operand (row l%16, key slots 8(l/16)..+7 in the permuted order) from the
// lane's own score-shaped registers.
template <typename T>
__device__ __forceinline__ typename Mma16<T>::Frag pack_rows(const f32x4 (&x)[2]) {
  typename Mma16<T>::Frag f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    f[u] = from_float<T>(x[0][u]);
    f[u + 4] = from_float<T>(x[1][u]);
  }
  return f;
}

// B operand of a 16x16x32 product for columns [d0, d0 + 16), read from a
// row-major tile X (stride LD) with two ds_read_tr16_b64: k slots 8(l/16) +
// {0..3} take rows r_lo + {0..3} and slots 8(l/16) + {4..7} rows r_hi +
// {0..3}, column d0 + l%16. Within a 16-lane group the instruction returns to
// lane i element i%4 of the 8 bytes that lanes 4j + i/4 (j = 0..3) address,
// so lane s addresses row r + s/4, columns d0 + 4(s%4)..+3.
template <typename T>
__device__ __forceinline__ typename Mma16<T>::Frag frag_tr_rows(const T* x, int r_lo, int r_hi, int d0) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef short s8 __attribute__((ext_vector_type(8)));
  const int s = threadIdx.x & 15;
  const T* p0 = x + (r_lo + (s >> 2)) * HaloMfma::LD + d0 + 4 * (s & 3);
  const T* p1 = x + (r_hi + (s >> 2)) * HaloMfma::LD + d0 + 4 * (s & 3);
  const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)p0);
  const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)p1);
  const s8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(typename Mma16<T>::Frag, v);
}

template <typename T>
__global__ __launch_bounds__(64) void halo_fwd_mfma_kernel(HaloArgs a) {
  typedef HaloMfma S;
  typedef Mma16<T> M;
  __shared__ __attribute__((aligned(16))) T qs[S::B_ * S::LD], ks[S::W * S::LD], vs[S::W * S::LD];
  const int lane = threadIdx.x, col = lane & 15, grp = lane >> 4;
  const int h = (int)(blockIdx.x % (unsigned)a.H);
  const int g = (int)((blockIdx.x / (unsigned)a.H) % (unsigned)a.G);
  const int bi = (int)(blockIdx.x / ((unsigned)a.H * (unsigned)a.G));
  const int64_t row0 = (int64_t)bi * (a.G + 1) * S::B_;
  {
    HaloLoads<T> L;
    load_unit<T, false>(a, row0, bi, h, g, L);
    store_unit<T, false>(a, L, g, qs, ks, vs, nullptr, nullptr);
  }
  __syncthreads();
  f32x4 p[2];
  window_tiles<T>(ks, qs, p);
  window_softmax(a, g, p);
  const typename M::Frag pa = pack_rows<T>(p);
  // the context rows go through the query tile (dead after the scores) and
  // leave as 16-byte stores
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    const f32x4 o = M::mma(pa, frag_tr_rows<T>(vs, 4 * grp, 16 + 4 * grp, 16 * dt), f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
    for (int r = 0; r < 4; ++r) qs[(4 * grp + r) * S::LD + 16 * dt + col] = from_float<T>(o[r]);
  }
  typedef typename Vec16<T>::type V;
  T* out = reinterpret_cast<T*>(a.out);
  const int64_t dim = (int64_t)a.H * S::HD;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int e = lane + 64 * t, row = e / 8, c = e % 8, tok = g * S::B_ + row;
    if (tok < a.n)
      *reinterpret_cast<V*>(out + ((int64_t)bi * a.n + tok) * dim + (int64_t)h * S::HD + c * 8) =
          *reinterpret_cast<const V*>(qs + row * S::LD + c * 8);
  }
}

// Two waves per SIMD (at most 256 registers): each wave's staging loads wait
// while the other computes (at stack_100m's shape 50 us, against 68 us at
// one wave per SIMD). Staging in two load phases keeps it within the limit
// without spills.
template <typename T>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void halo_bwd_mfma_kernel(HaloArgs a) {
  typedef HaloMfma S;
  typedef Mma16<T> M;
  typedef typename M::Frag F;
  __shared__ __attribute__((aligned(16))) T qs[S::B_ * S::LD], ks[S::W * S::LD], vs[S::W * S::LD];
  __shared__ __attribute__((aligned(16))) T dos[S::B_ * S::LD];
  __shared__ __attribute__((aligned(16))) T pts[S::B_ * S::LR], dsts[S::B_ * S::LR];
  __shared__ float delta[S::B_];
  const int lane = threadIdx.x, col = lane & 15, grp = lane >> 4;
  const int h = (int)(blockIdx.x % (unsigned)a.H);
  const int r = (int)((blockIdx.x / (unsigned)a.H) % (unsigned)(a.G + 1));
  const int bi = (int)(blockIdx.x / ((unsigned)a.H * (unsigned)(a.G + 1)));
  const int64_t row0 = (int64_t)bi * (a.G + 1) * S::B_;
  const int64_t dim = (int64_t)a.H * S::HD;
  T* dqkv = reinterpret_cast<T*>(a.dqkv);
  auto at = [&](int row, int slot, int d) { return ((row0 + row) * 3 + slot) * dim + (int64_t)h * S::HD + d; };
  // the 16 x 64 row tile x (stride LD, written by this wave) to block r's
  // rows of slot: 128 16-byte chunks, two per lane
  auto store_rows = [&](const T* x, int slot) {
    typedef typename Vec16<T>::type V;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int e = lane + 64 * t, row = e / 8, c = e % 8;
      *reinterpret_cast<V*>(dqkv + at(r * S::B_ + row, slot, c * 8)) =
          *reinterpret_cast<const V*>(x + row * S::LD + c * 8);
    }
  };
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  F fzero;
#pragma unroll
  for (int u = 0; u < 8; ++u) fzero[u] = from_float<T>(0.f);

  // rows 4(l/16) + i of block r, columns 16 dt + l%16: dv, and dk after the
  // rotary transpose, summed over both roles
  f32x4 dk[4], dv[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) dk[dt] = dv[dt] = zero;

  // role 0: own block of query block r-1; role 1: previous block of query
  // block r. (Loading the second role's tiles during the first role's
  // products measured slower: the registers held across them.)
  const int role0 = r == 0 ? 1 : 0, role1 = r == a.G ? 0 : 1;  // a.G >= 1: at least one role
#pragma unroll 1
  for (int role = role0; role <= role1; ++role) {
    const int g = role == 0 ? r - 1 : r;
    HaloLoads<T> L;
    // two load phases (queries and keys, then values, dO and O) keep fewer
    // registers in flight; the other wave on the SIMD covers the latency
    load_unit<T, true, 1>(a, row0, bi, h, g, L);  // registers only: before the barrier
    __syncthreads();
    store_unit<T, true, 1>(a, L, g, qs, ks, vs, dos, delta);
    load_unit<T, true, 2>(a, row0, bi, h, g, L);
    store_unit<T, true, 2>(a, L, g, qs, ks, vs, dos, delta);
    __syncthreads();
    f32x4 p[2], ds[2];
    window_tiles<T>(ks, qs, p);
    window_softmax(a, g, p);
    window_tiles<T>(vs, dos, ds);  // dP^T
    const float dl = delta[col];
#pragma unroll
    for (int t = 0; t < 2; ++t) ds[t] = p[t] * (ds[t] - dl);
    if (role == 0) {
      // dq of block r = scale dS K, through the query rotary transpose; the
      // rows go through LDS (the V rows are dead once dP^T is formed) and
      // leave as 16-byte stores
      const F da = pack_rows<T>(ds);
      f32x4 y[4];
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) y[dt] = M::mma(da, frag_tr_rows<T>(ks, 4 * grp, 16 + 4 * grp, 16 * dt), zero);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 4 * grp + i, d = 16 * dt + col;
          const float cs = a.cos_t[(S::B_ + row) * S::HALF + d], sn = a.sin_t[(S::B_ + row) * S::HALF + d];
          const float lo = a.scale * y[dt][i], hi = a.scale * y[dt + 2][i];
          vs[row * S::LD + d] = from_float<T>(lo * cs + hi * sn);
          vs[row * S::LD + d + S::HALF] = from_float<T>(hi * cs - lo * sn);
        }
      }
      store_rows(vs, 0);
    }
    // this role's window keys kk0 + j are block r's rows j
    const int th = role == 0 ? 1 : 0, kk0 = 16 * th;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pts[(4 * grp + i) * S::LR + col] = from_float<T>(p[th][i]);
      dsts[(4 * grp + i) * S::LR + col] = from_float<T>(ds[th][i]);
    }
    __syncthreads();
    const bool kin = grp < 2;  // k slots 0..15: the 16 query rows
    const F pa = kin ? *reinterpret_cast<const F*>(pts + col * S::LR + 8 * grp) : fzero;
    const F sa = kin ? *reinterpret_cast<const F*>(dsts + col * S::LR + 8 * grp) : fzero;
    const int rb = 8 * (grp & 1);  // lanes 32..63 read rows 0..15 too, then use zeros
    f32x4 kt[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const F ob_r = frag_tr_rows<T>(dos, rb, rb + 4, 16 * dt), qb_r = frag_tr_rows<T>(qs, rb, rb + 4, 16 * dt);
      const F ob = kin ? ob_r : fzero, qb = kin ? qb_r : fzero;
      dv[dt] = M::mma(pa, ob, dv[dt]);
      kt[dt] = M::mma(sa, qb, zero);
    }
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kk = kk0 + 4 * grp + i, d = 16 * dt + col;
        const float cs = a.cos_t[kk * S::HALF + d], sn = a.sin_t[kk * S::HALF + d];
        const float lo = a.scale * kt[dt][i], hi = a.scale * kt[dt + 2][i];
        dk[dt][i] += lo * cs + hi * sn;
        dk[dt + 2][i] += hi * cs - lo * sn;
      }
    }
  }
  // dk, dv (and the zero dq of block 0) through the Q and dO row tiles,
  // free after the last role's products
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * grp + i, d = 16 * dt + col;
      qs[row * S::LD + d] = from_float<T>(dk[dt][i]);
      dos[row * S::LD + d] = from_float<T>(dv[dt][i]);
    }
  }
  store_rows(qs, 1);
  store_rows(dos, 2);
  if (r == 0) {
    typedef typename Vec16<T>::type V;
    V z;
#pragma unroll
    for (int u = 0; u < 8; ++u) z[u] = from_float<T>(0.f);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int e = lane + 64 * t;
      *reinterpret_cast<V*>(dqkv + at(e / 8, 0, (e % 8) * 8)) = z;
    }
  }
}

// Instantiated shapes: the reference configurations use b = 16 (head_dim 64
// at stack_100m); every (b, hd) below fits the backward's LDS in 64 KiB.
template <typename T, bool BWD>
hipError_t dispatch(const HaloArgs& a, hipStream_t s) {
  const unsigned units = (unsigned)((int64_t)a.B * (BWD ? a.G + 1 : a.G) * a.H);
  auto go = [&]<int B_, int HD>() {
    auto note = [&](const void* f, const char* name) {
      note_launch(f, {name, dtype_code<T>(), HD, B_, B_, 2 * B_, 1, 1, units, "unit"});
    };
    if constexpr (HD == 64 && B_ == 16 && sizeof(T) == 2) {
      if constexpr (BWD) {
        note((const void*)&halo_bwd_mfma_kernel<T>, "halo_bwd_mfma");
        hipLaunchKernelGGL((halo_bwd_mfma_kernel<T>), dim3(units), dim3(64), 0, s, a);
      } else {
        note((const void*)&halo_fwd_mfma_kernel<T>, "halo_fwd_mfma");
        hipLaunchKernelGGL((halo_fwd_mfma_kernel<T>), dim3(units), dim3(64), 0, s, a);
      }
    } else if constexpr (HD == 64) {
      if constexpr (BWD) {
        note((const void*)&halo_bwd64_kernel<T, B_>, "halo_bwd64");
        hipLaunchKernelGGL((halo_bwd64_kernel<T, B_>), dim3(units), dim3(64), 0, s, a);
      } else {
        note((const void*)&halo_fwd64_kernel<T, B_>, "halo_fwd64");
        hipLaunchKernelGGL((halo_fwd64_kernel<T, B_>), dim3(units), dim3(64), 0, s, a);
      }
    } else {
      if constexpr (BWD) {
        note((const void*)&halo_bwd_kernel<T, B_, HD>, "halo_bwd");
        hipLaunchKernelGGL((halo_bwd_kernel<T, B_, HD>), dim3(units), dim3(64), 0, s, a);
      } else {
        note((const void*)&halo_fwd_kernel<T, B_, HD>, "halo_fwd");
        hipLaunchKernelGGL((halo_fwd_kernel<T, B_, HD>), dim3(units), dim3(64), 0, s, a);
      }
    }
    return hipGetLastError();
  };
#define ST_HALO_CASE(BB, DD) \
  if (a.b == BB && a.hd == DD) return go.template operator()<BB, DD>();
  ST_HALO_CASE(4, 32) ST_HALO_CASE(4, 64) ST_HALO_CASE(4, 128)
  ST_HALO_CASE(8, 32) ST_HALO_CASE(8, 64) ST_HALO_CASE(8, 128)
  ST_HALO_CASE(16, 32) ST_HALO_CASE(16, 64) ST_HALO_CASE(16, 128)
  ST_HALO_CASE(32, 32)
#undef ST_HALO_CASE
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t launch_t(bool bwd, const HaloArgs& a, hipStream_t s) {
  return bwd ? dispatch<T, true>(a, s) : dispatch<T, false>(a, s);
}

hipError_t launch(int dtype, bool bwd, const HaloArgs& a, hipStream_t s) {
  switch (dtype) {
    case 2: return launch_t<bf16>(bwd, a, s);
    case 1: return launch_t<f16>(bwd, a, s);
    default: return launch_t<float>(bwd, a, s);
  }
}

}  // namespace

bool halo_supported(int b, int hd) {
  return ((b == 4 || b == 8 || b == 16) && (hd == 32 || hd == 64 || hd == 128)) || (b == 32 && hd == 32);
}

hipError_t launch_halo_fwd(int dtype, const HaloArgs& a, hipStream_t stream) { return launch(dtype, false, a, stream); }
hipError_t launch_halo_bwd(int dtype, const HaloArgs& a, hipStream_t stream) { return launch(dtype, true, a, stream); }

}  // namespace st
