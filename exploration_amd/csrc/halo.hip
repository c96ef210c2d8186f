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

template <int B_, int HD>
constexpr size_t bwd_lds() {
  typedef HaloShape<B_, HD> S;
  return sizeof(float) * (7 * B_ * S::LD + 2 * B_ * S::PS + B_);
}

// Instantiated shapes: the reference configurations use b = 16 (head_dim 64
// at stack_100m); every (b, hd) below fits the backward's LDS in 64 KiB.
template <typename T, bool BWD>
hipError_t dispatch(const HaloArgs& a, hipStream_t s) {
  const unsigned units = (unsigned)((int64_t)a.B * (BWD ? a.G + 1 : a.G) * a.H);
  auto go = [&]<int B_, int HD>() {
    if constexpr (BWD) hipLaunchKernelGGL((halo_bwd_kernel<T, B_, HD>), dim3(units), dim3(64), 0, s, a);
    else hipLaunchKernelGGL((halo_fwd_kernel<T, B_, HD>), dim3(units), dim3(64), 0, s, a);
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

size_t halo_lds_bytes(int b, int hd) {
  if (!halo_supported(b, hd)) return 0;
  if (b == 32) return bwd_lds<32, 32>();
  const int w = 2 * b;
  return sizeof(float) * (7 * b * (hd + 1) + 2 * b * (w + 1) + b);
}

hipError_t launch_halo_fwd(int dtype, const HaloArgs& a, hipStream_t stream) { return launch(dtype, false, a, stream); }
hipError_t launch_halo_bwd(int dtype, const HaloArgs& a, hipStream_t stream) { return launch(dtype, true, a, stream); }

}  // namespace st
