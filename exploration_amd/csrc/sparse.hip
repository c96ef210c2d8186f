// Paged sparse top-k inference forward (gfx950): block scores, exact top-k
// selection and the gated sparse read.
//
// Semantics follow st/ops/sparse.py:15-174 and st/ops/kernels/sparse.py:9-113:
//   s_j = logsumexp_{i in block j} q.k_i/sqrt(D) for visible blocks
//   (j < p//b - 1, block complete inside the KV range), -inf otherwise;
//   log Z_R = logsumexp_j s_j; ids = top-k of s (descending, ties by
//   ascending block id, -1 for -inf); the output is the softmax over the
//   local window (blocks p//b-1 and p//b, up to p) with logits a_i and the
//   selected blocks with logits a_i + s_j - log Z_R.
//
// sparse_scores: one wave per (batch, head, 128-key chunk); S^T = K Q^T on
//   MFMA with K fragments loaded straight from HBM (each key read once per
//   32 queries), block logsumexp reduced in-lane.
// sparse_select: one workgroup per (batch, query, head) row; exact radix
//   select on the 64-bit key (ordered score, ~block id), then a rank sort.
// sparse_pop: one wave per (row, block slot); online softmax over the block's
//   tokens with coalesced 16-byte loads; sparse_merge combines the slots.
#include "report.h"
#include "sparse.h"
#include "tile.h"

namespace st {

// Token-row addressing of the KV view: pointer to token `t` (relative to
// token_offset) of head h, and the element stride between consecutive tokens
// of the same block (blocks never straddle pages).
template <typename T, bool PAGED>
__device__ __forceinline__ const T* kv_token(const KvView& kv, const T* base, int bi, int64_t t, int h,
                                             int H, int D) {
  if constexpr (PAGED) {
    // token counts stay below 2^32 (checked by the ABI): 32-bit division
    const uint32_t pt = (uint32_t)kv.page_tokens;
    const uint32_t lp = (uint32_t)t / pt;
    const int64_t page = kv.page_table[(int64_t)bi * kv.pages_per_seq + lp];
    return base + ((page * H + h) * (int64_t)pt + ((uint32_t)t - lp * pt)) * D;
  } else {
    return base + (((int64_t)bi * kv.n_tokens + t) * H + h) * D;
  }
}

template <bool PAGED> __device__ __forceinline__ int64_t kv_stride(int H, int D) {
  return PAGED ? (int64_t)D : (int64_t)H * D;
}

// N consecutive elements [d, d+N) of a row of D elements, zero past D. Rows
// whose length is a multiple of N are N-aligned and take one vector load;
// other head dimensions (not a multiple of 8) load element by element.
template <typename T, typename F, int N>
__device__ __forceinline__ F load_row_elems(const T* p, int d, int D) {
  if (D % N == 0) return d < D ? *reinterpret_cast<const F*>(p + d) : F{};
  F f;
#pragma unroll
  for (int e = 0; e < N; ++e) f[e] = d + e < D ? p[d + e] : T(0);
  return f;
}

// ---------------------------------------------------------------------------
template <typename T, int DP, bool PAGED>
__global__ __launch_bounds__(256) void sparse_scores_kernel(SparseArgs a) {
  typedef Mma<T> M;
  typedef typename M::Frag Frag;
  constexpr int NST = 4;  // 128 keys per wave
  constexpr int NKC = DP / M::KW;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int h = blockIdx.y, bi = blockIdx.z;
  const int64_t chunk = (int64_t)blockIdx.x * 4 + wave;
  const int64_t t0 = chunk * 128;  // first token of the chunk, relative to token_offset
  const int64_t n_tokens = a.kv.n_tokens;
  if (t0 >= n_tokens) return;
  const int b = a.block;
  const int64_t first_block = t0 / b;               // chunk-local block 0, relative
  const int nblk = 128 / b;                         // blocks in this chunk
  const int64_t stride = kv_stride<PAGED>(a.H, a.D);
  const T* kbase = reinterpret_cast<const T*>(a.kv.k);
  const T* qbase = reinterpret_cast<const T*>(a.q);

  for (int g0 = 0; g0 < a.Q; g0 += 32) {
    const int row = g0 + col;
    const bool row_in = row < a.Q;
    const int64_t p = row_in ? a.pos[(int64_t)bi * a.Q + row] : -1;
    // visible blocks are j < p//b - 1 (absolute); vis_lim is that limit in
    // the scores array's numbering (block 0 = token_offset / b)
    const int64_t vis_lim = p >= 0 ? p / b - 1 - a.id_base : -1;
    // skip the chunk when no row of this group sees any of its blocks
    float any = first_block < vis_lim ? 1.f : 0.f;
    any = fmaxf(any, other_half(any));
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) any = fmaxf(any, __shfl_xor(any, off, 64));

    float lse[NST][8];
    if (any > 0.f) {
      Frag qf[NKC];
      const T* qrow = qbase + (((int64_t)bi * a.Q + (row_in ? row : 0)) * a.H + h) * a.D;
#pragma unroll
      for (int c = 0; c < NKC; ++c) {
        const int d = c * M::KW + half * M::VEC;
        if constexpr (M::VEC == 1) qf[c] = (row_in && d < a.D) ? qrow[d] : 0.f;
        else qf[c] = row_in ? load_row_elems<T, Frag, M::VEC>(qrow, d, a.D) : Frag{};
      }
      f32x16 s[NST];
#pragma unroll
      for (int st = 0; st < NST; ++st) {
        int64_t t = t0 + 32 * st + col;
        t = t < n_tokens ? t : n_tokens - 1;  // rows past the range are loaded clamped and masked below
        const T* krow = kv_token<T, PAGED>(a.kv, kbase, bi, t, h, a.H, a.D);
        f32x16 acc = zero16();
#pragma unroll
        for (int c = 0; c < NKC; ++c) {
          const int d = c * M::KW + half * M::VEC;
          Frag kf;
          if constexpr (M::VEC == 1) kf = d < a.D ? krow[d] : 0.f;
          else kf = load_row_elems<T, Frag, M::VEC>(krow, d, a.D);
          acc = M::mma(kf, qf[c], acc);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t tok = t0 + 32 * st + c_row(r, half);
          acc[r] = tok < n_tokens ? acc[r] * a.scale_log2 : kNegInf;
        }
        s[st] = acc;
      }
      dispatch_logb(a.logb, [&]<int LOGB>() {
        float mx[NST][8], sm[NST][8];
        block_sums<NST, LOGB, OpMax>(s, mx);
#pragma unroll
        for (int st = 0; st < NST; ++st)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float m = mx[st][blk_slot<LOGB>(r)];
            s[st][r] = m == kNegInf ? 0.f : fast_exp2(s[st][r] - m);
          }
        block_sums<NST, LOGB, OpAdd>(s, sm);
#pragma unroll
        for (int st = 0; st < NST; ++st)
#pragma unroll
          for (int j = 0; j < 8; ++j)
            lse[st][j] = (j < BlkSlots<LOGB>::n && sm[st][j] > 0.f) ? (mx[st][j] + fast_log2(sm[st][j])) * kLn2
                                                                   : kNegInf;
      });
    }
    if (!row_in) continue;
    float* out = a.scores + (((int64_t)bi * a.Q + row) * a.H + h) * a.n_blocks;
    dispatch_logb(a.logb, [&]<int LOGB>() {
      if (!BlkSlots<LOGB>::per_half && half != 0) return;
#pragma unroll
      for (int st = 0; st < NST; ++st) {
        if constexpr (LOGB >= 5) {
          if ((32 * st) % (1 << LOGB) != 0) continue;  // one write per block
        }
#pragma unroll
        for (int j = 0; j < BlkSlots<LOGB>::n; ++j) {
          const int bl = blk_index<LOGB>(st, j, half);
          if (bl >= nblk) continue;
          const int64_t rel = first_block + bl;
          if (rel >= a.n_blocks) continue;
          const bool complete = (rel + 1) * b <= n_tokens;
          const bool visible = complete && rel < vis_lim;
          out[rel] = visible ? lse[st][j] : kNegInf;
        }
      }
    });
  }
}

// Bandwidth-shaped variant for 16-bit KV with head_dim <= 128: each wave
// copies its 128-key chunk into LDS with coalesced asynchronous 16-byte
// loads (a 128-token page of one head is one contiguous 32 KiB read), then
// reads MFMA fragments from an XOR-swizzled layout (chunk c of key row r is
// stored at chunk c ^ 2*(r % (CPR/2)), so 8 consecutive rows hit distinct
// banks).
template <typename T, int DP, bool PAGED, int LOGB_T>
__global__ __launch_bounds__(64, 2) void sparse_scan_kernel(SparseArgs a) {
  typedef Mma<T> M;
  typedef typename M::Frag Frag;
  static_assert(sizeof(T) == 2 && DP <= 128, "16-bit, head_dim <= 128");
  constexpr int E = 8;           // elements per 16-byte chunk
  constexpr int CPR = DP / E;    // chunks per key row
  constexpr int SWZ = CPR / 2;
  constexpr int KEYS = 128;
  constexpr int NST = KEYS / 32;
  constexpr int NKC = DP / M::KW;
  constexpr int COPIES = KEYS * CPR / 64;
  // one wave per workgroup: workgroups on a CU run out of phase, so one
  // wave's copies overlap another's arithmetic
  __shared__ __attribute__((aligned(16))) T buf[KEYS * DP];
  const int lane = threadIdx.x & 63;
  const int col = lane & 31, half = lane >> 5;
  const int h = blockIdx.y, bi = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.x * KEYS;
  const int64_t n_tokens = a.kv.n_tokens;
  if (t0 >= n_tokens) return;
  const int b = a.block;
  const int64_t first_block = t0 / b;
  const int nblk = KEYS / b;
  const T* kbase = reinterpret_cast<const T*>(a.kv.k);
  const T* qbase = reinterpret_cast<const T*>(a.q);
  bool loaded = false;

  for (int g0 = 0; g0 < a.Q; g0 += 32) {
    const int row = g0 + col;
    const bool row_in = row < a.Q;
    const int64_t p = row_in ? a.pos[(int64_t)bi * a.Q + row] : -1;
    const int64_t vis_lim = p >= 0 ? p / b - 1 - a.id_base : -1;
    float any = first_block < vis_lim ? 1.f : 0.f;
    any = fmaxf(any, other_half(any));
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) any = fmaxf(any, __shfl_xor(any, off, 64));

    Frag qf[NKC];
    if (any > 0.f) {
      if (!loaded) {
        // Row pointers first (page lookups batched, one wait), then the
        // copies back to back. A chunk inside one page needs one lookup.
        constexpr int RPI = 64 / CPR;  // key rows per copy instruction
        const int last = (int)(n_tokens - 1 - t0);  // rows past the range are clamped
        if (!PAGED || a.kv.page_tokens % KEYS == 0) {
          const T* base = kv_token<T, PAGED>(a.kv, kbase, bi, t0, h, a.H, a.D);
          const int64_t stride = kv_stride<PAGED>(a.H, a.D);
#pragma unroll
          for (int it = 0; it < COPIES; ++it) {
            const int slot = it * 64 + lane;
            const int r = it * RPI + lane / CPR;
            int chunk = (slot % CPR) ^ (2 * (r % SWZ));
            if (chunk * E >= a.D) chunk = 0;  // padded columns: any finite data (q pads with zeros)
            async_copy16(base + (int64_t)(r < last ? r : last) * stride + chunk * E, buf + it * 64 * E);
          }
        } else {
          // pages shorter than the chunk: one lookup per copy (rare path)
          for (int it = 0; it < COPIES; ++it) {
            const int slot = it * 64 + lane;
            const int r = it * RPI + lane / CPR;
            int chunk = (slot % CPR) ^ (2 * (r % SWZ));
            if (chunk * E >= a.D) chunk = 0;
            async_copy16(kv_token<T, PAGED>(a.kv, kbase, bi, t0 + (r < last ? r : last), h, a.H, a.D) + chunk * E,
                         buf + it * 64 * E);
          }
        }
        loaded = true;
      }
      const T* qrow = qbase + (((int64_t)bi * a.Q + (row_in ? row : 0)) * a.H + h) * a.D;
#pragma unroll
      for (int c = 0; c < NKC; ++c) {
        const int d = c * M::KW + half * M::VEC;
        if constexpr (M::VEC == 1) qf[c] = (row_in && d < a.D) ? qrow[d] : 0.f;
        else qf[c] = row_in ? load_row_elems<T, Frag, M::VEC>(qrow, d, a.D) : Frag{};
      }
      wait_vm();
    }
    float* out = a.scores + (((int64_t)bi * a.Q + (row_in ? row : 0)) * a.H + h) * a.n_blocks;
    // One 32-key subtile at a time; blocks wider than a subtile keep a
    // running (max, sum) across their subtiles.
    float run_m = kNegInf, run_s = 0.f;
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      f32x16 acc = zero16();
      if (any > 0.f) {
        const int r = 32 * st + col;
#pragma unroll
        for (int c = 0; c < NKC; ++c) {
          const int chunk = (2 * c + half) ^ (2 * (r % SWZ));
          acc = M::mma(*reinterpret_cast<const Frag*>(buf + r * DP + chunk * E), qf[c], acc);
        }
      }
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int64_t tok = t0 + 32 * st + c_row(rr, half);
        acc[rr] = tok < n_tokens ? acc[rr] * a.scale_log2 : kNegInf;
      }
      ([&]<int LOGB>() {
        auto emit = [&](int bl, float lse2) {
          if (bl >= nblk || !row_in) return;  // invisible blocks still get -inf
          const int64_t rel = first_block + bl;
          if (rel >= a.n_blocks) return;
          const bool visible = (rel + 1) * b <= n_tokens && rel < vis_lim;
          out[rel] = visible ? lse2 * kLn2 : kNegInf;
        };
        if constexpr (LOGB >= 5) {
          float m = acc[0];
#pragma unroll
          for (int rr = 1; rr < 16; ++rr) m = fmaxf(m, acc[rr]);
          m = fmaxf(m, other_half(m));
          float sm = 0.f;
          if (m != kNegInf) {
#pragma unroll
            for (int rr = 0; rr < 16; ++rr) sm += fast_exp2(acc[rr] - m);
          }
          sm += other_half(sm);
          const float nm = fmaxf(run_m, m);
          if (nm != kNegInf)
            run_s = (run_m == kNegInf ? 0.f : run_s * fast_exp2(run_m - nm)) +
                    (m == kNegInf ? 0.f : sm * fast_exp2(m - nm));
          run_m = nm;
          constexpr int G = (1 << LOGB) / 32;
          if ((st + 1) % G == 0) {
            if (half == 0) emit((32 * st) >> LOGB, run_s > 0.f ? run_m + fast_log2(run_s) : kNegInf);
            run_m = kNegInf;
            run_s = 0.f;
          }
        } else {
          f32x16 x[1] = {acc};
          float mx[1][8], sm[1][8];
          block_sums<1, LOGB, OpMax>(x, mx);
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) {
            const float m = mx[0][blk_slot<LOGB>(rr)];
            x[0][rr] = m == kNegInf ? 0.f : fast_exp2(x[0][rr] - m);
          }
          block_sums<1, LOGB, OpAdd>(x, sm);
          if (!BlkSlots<LOGB>::per_half && half != 0) return;
#pragma unroll
          for (int j = 0; j < BlkSlots<LOGB>::n; ++j)
            emit(blk_index<LOGB>(st, j, half), sm[0][j] > 0.f ? mx[0][j] + fast_log2(sm[0][j]) : kNegInf);
        }
      }).template operator()<LOGB_T>();
    }
  }
  if (loaded) wait_vm();  // no copy may still target LDS when the wave ends
}

// ---------------------------------------------------------------------------
// Direct variant for 16-bit KV, head_dim a multiple of 32 and <= 128:
// v_mfma_f32_16x16x32 with S^T = K Q^T for 16 queries at a time. Lane l
// loads 16 bytes of key row l%16 at dims 32c + 8*(l/16), so the four lanes
// of a key read 64 contiguous bytes per instruction, straight into
// registers: the bytes in flight are bounded by registers, not by LDS. A
// score row lives in lanes j, j+16, j+32, j+48 (4 keys each per 16-key
// subtile); block reductions are in-lane plus two cross-lane steps.
template <typename T, int DP, bool PAGED, int LOGB>
__global__ __launch_bounds__(256, 2) void sparse_scan16_kernel(SparseArgs a) {
  typedef Mma16<T> M;
  typedef typename M::Frag Frag;
  constexpr int KEYS = 128;             // keys per wave
  constexpr int NS = KEYS / 16;         // 16-key subtiles
  constexpr int NKC = DP / 32;          // contraction chunks
  constexpr int B = 1 << LOGB;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  // heads vary fastest across workgroups: the H head slices of a page are
  // read by neighbouring workgroups at about the same time
  const int h = (int)(blockIdx.x % (uint32_t)a.H), bi = blockIdx.z;
  const int64_t t0 = ((int64_t)(blockIdx.x / (uint32_t)a.H) * 4 + wave) * KEYS;
  const int64_t n_tokens = a.kv.n_tokens;
  if (t0 >= n_tokens) return;
  const int64_t first_block = t0 >> LOGB;
  const T* kbase = reinterpret_cast<const T*>(a.kv.k);
  const T* qbase = reinterpret_cast<const T*>(a.q);
  const int64_t stride = kv_stride<PAGED>(a.H, a.D);
  const int last = (int)(n_tokens - 1 - t0);
  // key row pointers of this lane's 8 subtiles (one page lookup per chunk
  // when pages hold whole chunks)
  const T* krow[NS];
  if (!PAGED || a.kv.page_tokens % KEYS == 0) {
    const T* base = kv_token<T, PAGED>(a.kv, kbase, bi, t0, h, a.H, a.D);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int r = 16 * s + j;
      krow[s] = base + (int64_t)(r < last ? r : last) * stride;
    }
  } else {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int r = 16 * s + j;
      krow[s] = kv_token<T, PAGED>(a.kv, kbase, bi, t0 + (r < last ? r : last), h, a.H, a.D);
    }
  }
  bool loaded = false;
  Frag kf[NS][NKC];
  for (int g0 = 0; g0 < a.Q; g0 += 16) {
    const int row = g0 + j;
    const bool row_in = row < a.Q;
    const int64_t p = row_in ? a.pos[(int64_t)bi * a.Q + row] : -1;
    const int64_t vis_lim = p >= 0 ? p / (int64_t)B - 1 - a.id_base : -1;
    float any = first_block < vis_lim ? 1.f : 0.f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) any = fmaxf(any, __shfl_xor(any, off, 64));
    float* out = a.scores + (((int64_t)bi * a.Q + (row_in ? row : 0)) * a.H + h) * a.n_blocks;
    f32x4 acc[NS];
    if (any > 0.f) {
      if (!loaded) {
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
          for (int c = 0; c < NKC; ++c) {
            const int d = 32 * c + 8 * g;
            kf[s][c] = d < a.D ? *reinterpret_cast<const Frag*>(krow[s] + d) : Frag{};
          }
        loaded = true;
      }
      Frag qf[NKC];
      const T* qrow = qbase + (((int64_t)bi * a.Q + (row_in ? row : 0)) * a.H + h) * a.D;
#pragma unroll
      for (int c = 0; c < NKC; ++c) {
        const int d = 32 * c + 8 * g;
        qf[c] = (row_in && d < a.D) ? *reinterpret_cast<const Frag*>(qrow + d) : Frag{};
      }
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        f32x4 c4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NKC; ++c) c4 = M::mma(kf[s][c], qf[c], c4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t tok = t0 + 16 * s + 4 * g + r;
          c4[r] = tok < n_tokens ? c4[r] * a.scale_log2 : kNegInf;
        }
        acc[s] = c4;
      }
    } else {
#pragma unroll
      for (int s = 0; s < NS; ++s) acc[s] = f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
    }
    if (!row_in) continue;
    auto emit = [&](int bl, float lse2) {
      const int64_t rel = first_block + bl;
      if (rel >= a.n_blocks) return;
      const bool visible = (rel + 1) * B <= n_tokens && rel < vis_lim;
      out[rel] = visible ? lse2 * kLn2 : kNegInf;
    };
    if constexpr (B >= 16) {
      // a block = B/16 whole subtiles; lanes g hold 4 keys of each
      constexpr int SPB = B / 16;
#pragma unroll
      for (int b0 = 0; b0 < NS; b0 += SPB) {
        float m = kNegInf;
#pragma unroll
        for (int s = b0; s < b0 + SPB; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) m = fmaxf(m, acc[s][r]);
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        m = fmaxf(m, __shfl_xor(m, 32, 64));
        float sm = 0.f;
        if (m != kNegInf) {
#pragma unroll
          for (int s = b0; s < b0 + SPB; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r) sm += fast_exp2(acc[s][r] - m);
        }
        sm += __shfl_xor(sm, 16, 64);
        sm += __shfl_xor(sm, 32, 64);
        if (g == 0) emit(b0 / SPB, sm > 0.f ? m + fast_log2(sm) : kNegInf);
      }
    } else if constexpr (B == 8) {
      // keys 8k..8k+7 of a subtile live in lane groups g = 2k, 2k+1
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        float m = fmaxf(fmaxf(acc[s][0], acc[s][1]), fmaxf(acc[s][2], acc[s][3]));
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        float sm = 0.f;
        if (m != kNegInf)
#pragma unroll
          for (int r = 0; r < 4; ++r) sm += fast_exp2(acc[s][r] - m);
        sm += __shfl_xor(sm, 16, 64);
        if ((g & 1) == 0) emit(2 * s + (g >> 1), sm > 0.f ? m + fast_log2(sm) : kNegInf);
      }
    } else {
      // blocks of 4 (one lane group) or 2 (half of one)
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int q0 = 0; q0 < 4; q0 += B) {
          float m = acc[s][q0];
#pragma unroll
          for (int r = 1; r < B; ++r) m = fmaxf(m, acc[s][q0 + r]);
          float sm = 0.f;
          if (m != kNegInf)
#pragma unroll
            for (int r = 0; r < B; ++r) sm += fast_exp2(acc[s][q0 + r] - m);
          emit((16 * s + 4 * g + q0) >> LOGB, sm > 0.f ? m + fast_log2(sm) : kNegInf);
        }
    }
  }
}

// ---------------------------------------------------------------------------
// Single-pass top-k for k <= 64: each wave streams a quarter of the row,
// keeps its running top-64 as one 64-bit key per lane (sorted descending
// across lanes), and only keys above the current 64th key are buffered and
// merged (bitonic sort of 64 + bitonic merge). The four wave lists are then
// merged by wave 0. Exact: keys are distinct (score bits, ~block id).
__device__ __forceinline__ uint64_t shfl_xor64(uint64_t x, int m) {
  const int lo = __shfl_xor((int)(uint32_t)x, m, 64);
  const int hi = __shfl_xor((int)(uint32_t)(x >> 32), m, 64);
  return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

__device__ __forceinline__ uint64_t wave_sort_asc(uint64_t x, int lane) {
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const uint64_t y = shfl_xor64(x, j);
      const bool keep_min = ((lane & j) == 0) == ((lane & k) == 0);
      x = keep_min ? (x < y ? x : y) : (x > y ? x : y);
    }
  return x;
}

// r sorted descending, c sorted ascending: the top 64 of both, descending.
__device__ __forceinline__ uint64_t wave_merge_desc(uint64_t r, uint64_t c, int lane) {
  uint64_t x = r > c ? r : c;
#pragma unroll
  for (int j = 32; j > 0; j >>= 1) {
    const uint64_t y = shfl_xor64(x, j);
    x = ((lane & j) == 0) ? (x > y ? x : y) : (x < y ? x : y);
  }
  return x;
}

__device__ __forceinline__ uint64_t lane63(uint64_t x) {
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)x, 63);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint32_t ordered_bits(float x);

__global__ __launch_bounds__(256) void sparse_select64_kernel(int64_t n_blocks, int topk, int64_t id_base,
                                                              const float* scores, int64_t* ids, float* top,
                                                              float* log_zr) {
  __shared__ uint64_t cand[4][128];
  __shared__ uint64_t lists[4][64];
  __shared__ float red_m[4], red_s[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;
  const float* s = scores + row * n_blocks;
  const int64_t seg = (((n_blocks + 3) / 4) + 63) / 64 * 64;
  const int64_t lo = wave * seg;
  const int64_t hi = lo + seg < n_blocks ? lo + seg : n_blocks;
  float m = kNegInf, sum = 0.f;
  uint64_t best = 0, theta = 0;
  int cnt = 0;
  auto flush = [&](int take) {
    uint64_t x = lane < take ? cand[wave][lane] : 0;
    x = wave_sort_asc(x, lane);
    best = wave_merge_desc(best, x, lane);
    theta = lane63(best);
  };
  // Batches of 32 scores per lane. Each batch first merges the 64 lane
  // maxima (64 distinct keys, so the 64th best key of the batch is at least
  // their minimum); afterwards only keys above the running 64th key are
  // buffered and merged.
  constexpr int BATCH = 32;
  auto key_at = [&](float x, int64_t i) -> uint64_t {
    return ((uint64_t)ordered_bits(x) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
  };
  for (int64_t base0 = lo; base0 < hi; base0 += 64 * BATCH) {
    float xs[BATCH];
#pragma unroll
    for (int q = 0; q < BATCH; ++q) {
      const int64_t i = base0 + 64 * q + lane;
      xs[q] = i < hi ? s[i] : kNegInf;
    }
    uint64_t kmax = 0;
#pragma unroll
    for (int q = 0; q < BATCH; ++q) {
      const int64_t i = base0 + 64 * q + lane;
      const float x = xs[q];
      if (x > m) {
        sum = (m == kNegInf ? 0.f : sum * __expf(m - x)) + 1.f;
        m = x;
      } else if (x != kNegInf) {
        sum += __expf(x - m);
      }
      const uint64_t key = i < hi ? key_at(x, i) : 0;
      kmax = key > kmax ? key : kmax;
    }
    best = wave_merge_desc(best, wave_sort_asc(kmax, lane), lane);
    theta = lane63(best);
#pragma unroll
    for (int q = 0; q < BATCH; ++q) {
      const int64_t i = base0 + 64 * q + lane;
      const uint64_t key = i < hi ? key_at(xs[q], i) : 0;
      const bool pass = key > theta && key != kmax;
      const uint64_t mask = __ballot(pass);
      if (mask == 0) continue;
      const int rank = __popcll(mask & ((1ull << lane) - 1ull));
      if (pass) cand[wave][cnt + rank] = key;
      cnt += __popcll(mask);
      if (cnt >= 64) {
        flush(64);
        const int rest = cnt - 64;
        uint64_t moved = lane < rest ? cand[wave][64 + lane] : 0;
        if (lane < rest) cand[wave][lane] = moved;
        cnt = rest;
      }
    }
  }
  if (cnt > 0) flush(cnt);
  lists[wave][lane] = best;
  // per-wave logsumexp partial
  float mw = m;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mw = fmaxf(mw, __shfl_xor(mw, off, 64));
  float sw = (m == kNegInf) ? 0.f : sum * __expf(m - mw);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sw += __shfl_xor(sw, off, 64);
  if (lane == 0) { red_m[wave] = mw; red_s[wave] = sw; }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 1; w < 4; ++w) best = wave_merge_desc(best, lists[w][63 - lane], lane);
  if (lane < topk) {
    float sc = kNegInf;
    int64_t id = -1;
    if (best != 0) {
      const uint32_t ob = (uint32_t)(best >> 32);
      const uint32_t u = (ob & 0x80000000u) ? (ob & 0x7fffffffu) : ~ob;
      sc = __uint_as_float(u);
      if (sc != kNegInf) id = (int64_t)(0xffffffffu - (uint32_t)(best & 0xffffffffu)) + id_base;
    }
    top[row * topk + lane] = sc;
    ids[row * topk + lane] = id;
  }
  if (lane == 0) {
    const float mm = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
    float tot = 0.f;
    if (mm != kNegInf)
      for (int w = 0; w < 4; ++w) tot += red_m[w] == kNegInf ? 0.f : red_s[w] * __expf(red_m[w] - mm);
    log_zr[row] = (mm == kNegInf || !(tot > 0.f)) ? kNegInf : mm + __logf(tot);
  }
}

// ---------------------------------------------------------------------------
// Radix top-k for k <= 64 and rows of at most NT*VMAX blocks: the row's
// 64-bit keys (ordered score bits, ~block id: all distinct) stay in
// registers; the bytes shared by every key (the row's min and max key agree
// on them) are skipped, then one byte per pass: a 256-bin LDS histogram of
// the keys that still match the prefix, a suffix scan, and the bin that
// holds the k-th largest key. The pass ends early when that bin's keys are
// all selected. The selected keys are compacted and rank-sorted.
template <int NT, int VMAX>
__global__ __launch_bounds__(NT) void sparse_select_radix_kernel(int64_t n_blocks, int topk, int64_t id_base,
                                                                 const float* scores, int64_t* ids, float* top,
                                                                 float* log_zr) {
  constexpr int NW = NT / 64;
  __shared__ uint32_t hist[256];
  __shared__ uint32_t wsum[4];
  __shared__ uint64_t sel[64];
  __shared__ uint64_t red_k[2][NW];
  __shared__ float red_m[NW], red_s[NW];
  __shared__ uint32_t ctrl[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const float* s = scores + row * n_blocks;
  const int n = (int)n_blocks;
  if (tid == 0) ctrl[3] = 0;
  uint64_t key[VMAX];
  float m = kNegInf, sum = 0.f;
  uint64_t kmax = 0, kmin = ~0ull;
  // unconditional loads (clamped index): all VMAX in flight together
  float xs[VMAX];
#pragma unroll
  for (int v = 0; v < VMAX; ++v) xs[v] = s[tid + NT * v < n ? tid + NT * v : n - 1];
#pragma unroll
  for (int v = 0; v < VMAX; ++v) {
    const int i = tid + NT * v;
    const float x = i < n ? xs[v] : kNegInf;
    key[v] = ((uint64_t)ordered_bits(x) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
    if (i < n) {
      kmax = key[v] > kmax ? key[v] : kmax;
      kmin = key[v] < kmin ? key[v] : kmin;
    }
    if (x > m) {
      sum = (m == kNegInf ? 0.f : sum * __expf(m - x)) + 1.f;
      m = x;
    } else if (x != kNegInf) {
      sum += __expf(x - m);
    }
  }
  // row logsumexp and the key range
  float mw = m;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mw = fmaxf(mw, __shfl_xor(mw, off, 64));
  float sw = (m == kNegInf) ? 0.f : sum * __expf(m - mw);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    sw += __shfl_xor(sw, off, 64);
    const uint64_t a = shfl_xor64(kmax, off), b = shfl_xor64(kmin, off);
    kmax = a > kmax ? a : kmax;
    kmin = b < kmin ? b : kmin;
  }
  if (lane == 0) {
    red_m[wave] = mw;
    red_s[wave] = sw;
    red_k[0][wave] = kmax;
    red_k[1][wave] = kmin;
  }
  __syncthreads();
  kmax = red_k[0][0];
  kmin = red_k[1][0];
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    kmax = red_k[0][w] > kmax ? red_k[0][w] : kmax;
    kmin = red_k[1][w] < kmin ? red_k[1][w] : kmin;
  }
  if (tid == 0) {
    float mm = red_m[0];
    for (int w = 1; w < NW; ++w) mm = fmaxf(mm, red_m[w]);
    float tot = 0.f;
    if (mm != kNegInf)
      for (int w = 0; w < NW; ++w) tot += red_m[w] == kNegInf ? 0.f : red_s[w] * __expf(red_m[w] - mm);
    log_zr[row] = (mm == kNegInf || !(tot > 0.f)) ? kNegInf : mm + __logf(tot);
  }
  // select: keys whose top (64 - shift) bits are >= prefix
  int shift = 64;
  uint64_t prefix = 0;
  if (n > topk) {
    const uint64_t diff = kmax ^ kmin;  // nonzero: n >= 2 distinct keys
    const int common = __builtin_clzll(diff) & ~7;
    shift = 64 - common;
    prefix = common ? (kmax >> shift) : 0;
    uint32_t kk = (uint32_t)topk;
    while (true) {
      shift -= 8;
      if (tid < 256) hist[tid] = 0;
      __syncthreads();
      // Scores crowd into few bins (often one), and same-address LDS atomics
      // serialise: the lanes sharing the first two leaders' digits add their
      // count with one atomic each, the rest add one by one.
#pragma unroll
      for (int v = 0; v < VMAX; ++v) {
        bool match = tid + NT * v < n && (shift + 8 == 64 || (key[v] >> (shift + 8)) == prefix);
        const uint32_t digit = (uint32_t)(key[v] >> shift) & 255u;
#pragma unroll
        for (int round = 0; round < 2; ++round) {
          const uint64_t act = __ballot(match);
          if (act == 0) break;
          const int leader = __builtin_ctzll(act);
          const uint32_t ld = (uint32_t)__builtin_amdgcn_readlane((int)digit, leader);
          const bool same = match && digit == ld;
          const uint64_t group = __ballot(same);
          if (lane == leader) atomicAdd(&hist[ld], (uint32_t)__popcll(group));
          match = match && !same;
        }
        if (match) atomicAdd(&hist[digit], 1u);
      }
      __syncthreads();
      // suffix sums: thread t < 256 holds bin 255 - t
      uint32_t hv = 0, incl = 0;
      if (tid < 256) {
        hv = hist[255 - tid];
        incl = hv;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const uint32_t y = __shfl_up(incl, off, 64);
          if (lane >= off) incl += y;
        }
        if (lane == 63) wsum[wave] = incl;
      }
      __syncthreads();
      if (tid < 256) {
        for (int w = 0; w < wave; ++w) incl += wsum[w];
        const uint32_t above = incl - hv;
        if (above < kk && incl >= kk) {
          ctrl[0] = 255u - (uint32_t)tid;
          ctrl[1] = kk - above;
          ctrl[2] = hv;
        }
      }
      __syncthreads();
      const uint32_t d = ctrl[0], hd = ctrl[2];
      kk = ctrl[1];
      prefix = (prefix << 8) | d;
      if (hd == kk || shift == 0) break;
    }
  }
  // compaction: slots within the wave from ballots, one atomic per wave
  uint32_t slot[VMAX];
  uint32_t wave_cnt = 0;
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int v = 0; v < VMAX; ++v) {
    const bool take = tid + NT * v < n && (shift == 64 || (key[v] >> shift) >= prefix);
    const uint64_t mask = __ballot(take);
    slot[v] = take ? wave_cnt + (uint32_t)__popcll(mask & below) : ~0u;
    wave_cnt += (uint32_t)__popcll(mask);
  }
  if (wave_cnt) {
    uint32_t base = 0;
    if (lane == 0) base = atomicAdd(&ctrl[3], wave_cnt);
    base = (uint32_t)__builtin_amdgcn_readlane((int)base, 0);
#pragma unroll
    for (int v = 0; v < VMAX; ++v)
      if (slot[v] != ~0u) sel[base + slot[v]] = key[v];
  }
  __syncthreads();
  if (wave != 0) return;
  const int cnt = (int)ctrl[3];
  if (lane < cnt) {
    const uint64_t mine = sel[lane];
    int rank = 0;
    for (int j = 0; j < cnt; ++j) rank += sel[j] > mine;
    const uint32_t ob = (uint32_t)(mine >> 32);
    const float sc = __uint_as_float((ob & 0x80000000u) ? (ob & 0x7fffffffu) : ~ob);
    top[row * topk + rank] = sc;
    ids[row * topk + rank] = sc != kNegInf ? (int64_t)(0xffffffffu - (uint32_t)(mine & 0xffffffffu)) + id_base : -1;
  } else if (lane < topk) {
    top[row * topk + lane] = kNegInf;
    ids[row * topk + lane] = -1;
  }
}

// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t ordered_bits(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ __launch_bounds__(256) void sparse_select_kernel(int64_t n_blocks, int topk, int64_t id_base,
                                                            const float* scores, int64_t* ids, float* top,
                                                            float* log_zr) {
  __shared__ uint32_t hist[256];
  __shared__ float red[8];
  __shared__ uint64_t sel_key[4096];
  __shared__ int sel_count;
  __shared__ uint64_t prefix_sh;
  __shared__ int64_t remaining_sh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const float* s = scores + row * n_blocks;

  // log Z_R = logsumexp of the row
  float mx = kNegInf;
  for (int64_t i = tid; i < n_blocks; i += 256) mx = fmaxf(mx, s[i]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float sum = 0.f;
  if (mx != kNegInf)
    for (int64_t i = tid; i < n_blocks; i += 256) sum += __expf(s[i] - mx);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  if (lane == 0) red[4 + wave] = sum;
  __syncthreads();
  if (tid == 0) {
    const float tot = red[4] + red[5] + red[6] + red[7];
    log_zr[row] = (mx == kNegInf || !(tot > 0.f)) ? kNegInf : mx + __logf(tot);
  }

  // key = ordered score in the high word, inverted block id in the low word:
  // larger key = higher score, then lower id. All keys are distinct.
  auto key_of = [&](int64_t i) -> uint64_t {
    return ((uint64_t)ordered_bits(s[i]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
  };
  const int keep = (int64_t)topk < n_blocks ? topk : (int)n_blocks;
  uint64_t kth = 0;  // smallest selected key
  if ((int64_t)topk < n_blocks) {
    if (tid == 0) { prefix_sh = 0; remaining_sh = topk; }
    uint64_t mask = 0;
    for (int pass = 0; pass < 8; ++pass) {
      const int shift = 56 - 8 * pass;
      hist[tid] = 0;
      __syncthreads();
      const uint64_t prefix = prefix_sh;
      for (int64_t i = tid; i < n_blocks; i += 256) {
        const uint64_t k = key_of(i);
        if ((k & mask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        int64_t rem = remaining_sh;
        int d = 255;
        for (; d > 0; --d) {
          if ((int64_t)hist[d] >= rem) break;
          rem -= hist[d];
        }
        remaining_sh = rem;
        prefix_sh = prefix | ((uint64_t)d << shift);
      }
      mask |= (uint64_t)255 << shift;
      __syncthreads();
    }
    kth = prefix_sh;
  }

  // gather the selected keys, then rank them (descending)
  if (tid == 0) sel_count = 0;
  __syncthreads();
  for (int64_t i = tid; i < n_blocks; i += 256) {
    const uint64_t k = key_of(i);
    if (k >= kth) {
      const int slot = atomicAdd(&sel_count, 1);
      if (slot < 4096) sel_key[slot] = k;
    }
  }
  __syncthreads();
  const int cnt = sel_count < keep ? sel_count : keep;
  int64_t* ids_row = ids + row * topk;
  float* top_row = top + row * topk;
  for (int i = tid; i < cnt; i += 256) {
    const uint64_t k = sel_key[i];
    int rank = 0;
    for (int j = 0; j < cnt; ++j) rank += sel_key[j] > k ? 1 : 0;
    const uint32_t idx = 0xffffffffu - (uint32_t)(k & 0xffffffffu);
    const float sc = s[idx];
    top_row[rank] = sc;
    ids_row[rank] = sc == kNegInf ? -1 : (int64_t)idx + id_base;
  }
  for (int i = cnt + tid; i < topk; i += 256) {
    top_row[i] = kNegInf;
    ids_row[i] = -1;
  }
}

// ---------------------------------------------------------------------------
// Pop: wave = one block slot of one row. Slots 0 and 1 are the local blocks
// p//b - 1 and p//b, slot 2 + i is the i-th selected block.
template <typename T, int DP, bool PAGED>
__global__ __launch_bounds__(256) void sparse_pop_kernel(SparseArgs a) {
  typedef typename Vec16<T>::type V;
  constexpr int E = Vec16<T>::n;       // elements per 16-byte load
  constexpr int LPT = DP / E;          // lanes per token
  constexpr int TPI = 64 / LPT;        // tokens per load instruction
  __shared__ float part_m[4], part_l[4];
  __shared__ float part_o[4][DP];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;
  const int h = (int)(row % a.H);
  const int t = (int)((row / a.H) % a.Q);
  const int bi = (int)(row / ((int64_t)a.H * a.Q));
  const int slot = blockIdx.y * 4 + wave;
  const int b = a.block;
  const int64_t p = a.pos[(int64_t)bi * a.Q + t];
  const int g = lane / LPT;            // token within an instruction
  const int e0 = (lane % LPT) * E;     // first dimension of this lane

  int64_t blk = -1;
  float bias2 = 0.f;
  bool ok = p >= 0 && slot < a.topk + 2;
  if (ok) {
    if (slot < 2) {
      blk = p / b - 1 + slot;
    } else {
      blk = a.ids[row * a.topk + (slot - 2)];
      const float sc = a.top_scores[row * a.topk + (slot - 2)];
      float zr = a.log_zr[row];
      zr = zr == kNegInf ? 0.f : zr;
      ok = blk >= 0 && sc != kNegInf;
      bias2 = (sc - zr) * kLog2e;
    }
    ok = ok && blk >= 0;
  }
  // tokens [lo, hi) of this block that are readable: inside the KV range and <= p
  int64_t lo = 0, hi = 0;
  if (ok) {
    lo = blk * b;
    hi = lo + b;
    const int64_t r0 = a.kv.token_offset, r1 = a.kv.token_offset + a.kv.n_tokens;
    lo = lo > r0 ? lo : r0;
    hi = hi < r1 ? hi : r1;
    hi = hi < p + 1 ? hi : p + 1;
    if (hi <= lo) ok = false;
  }

  float q[E];
  {
    const T* qrow = reinterpret_cast<const T*>(a.q) + row * a.D;
    const V qv = load_row_elems<T, V, E>(qrow, e0, a.D);
#pragma unroll
    for (int e = 0; e < E; ++e) q[e] = to_float<T>(qv[e]) * a.scale_log2;
  }
  float m = kNegInf, l = 0.f, o[E];
#pragma unroll
  for (int e = 0; e < E; ++e) o[e] = 0.f;

  if (ok) {
    const int64_t stride = kv_stride<PAGED>(a.H, a.D);
    const int64_t tb = blk * b - a.kv.token_offset;  // block start, range-relative
    const int64_t tstart = (tb > 0 ? tb : 0);
    const T* kb = kv_token<T, PAGED>(a.kv, reinterpret_cast<const T*>(a.kv.k), bi, tstart, h, a.H, a.D);
    const T* vb = kv_token<T, PAGED>(a.kv, reinterpret_cast<const T*>(a.kv.v), bi, tstart, h, a.H, a.D);
    const int ntok = (int)(hi - lo);  // tokens from tstart on (lo == tstart + token_offset)
    constexpr int BATCH = 8;  // token rounds whose loads are in flight together
    for (int i00 = 0; i00 < ntok; i00 += TPI * BATCH) {
     V kvs[BATCH], vvs[BATCH];
#pragma unroll
     for (int j = 0; j < BATCH; ++j) {
       const int i = i00 + TPI * j + g;
       kvs[j] = V{};
       vvs[j] = V{};
       if (i < ntok) {
         kvs[j] = load_row_elems<T, V, E>(kb + (int64_t)i * stride, e0, a.D);
         vvs[j] = load_row_elems<T, V, E>(vb + (int64_t)i * stride, e0, a.D);
       }
     }
#pragma unroll
     for (int j = 0; j < BATCH; ++j) {
      const int i0 = i00 + TPI * j;
      if (i0 >= ntok) break;
      const int i = i0 + g;
      const bool valid = i < ntok;
      const V kv = kvs[j], vv = vvs[j];
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) dot += q[e] * to_float<T>(kv[e]);
#pragma unroll
      for (int off = 1; off < LPT; off <<= 1) dot += __shfl_xor(dot, off, 64);
      const float x = valid ? dot + bias2 : kNegInf;
      const float mn = fmaxf(m, x);
      if (mn != kNegInf) {
        const float alpha = fast_exp2(m - mn);
        const float pw = fast_exp2(x - mn);
        l = l * alpha + pw;
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = o[e] * alpha + pw * to_float<T>(vv[e]);
        m = mn;
      }
     }
    }
  }
  // merge the TPI token groups (lanes e0-aligned, differing in g)
#pragma unroll
  for (int off = LPT; off < 64; off <<= 1) {
    const float m2 = __shfl_xor(m, off, 64);
    const float l2 = __shfl_xor(l, off, 64);
    const float mn = fmaxf(m, m2);
    const float a1 = mn == kNegInf ? 0.f : fast_exp2(m - mn);
    const float a2 = mn == kNegInf ? 0.f : fast_exp2(m2 - mn);
    l = l * a1 + l2 * a2;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float o2 = __shfl_xor(o[e], off, 64);
      o[e] = o[e] * a1 + o2 * a2;
    }
    m = mn;
  }
  if (lane < LPT) {
#pragma unroll
    for (int e = 0; e < E; ++e) part_o[wave][e0 + e] = o[e];
    if (lane == 0) { part_m[wave] = m; part_l[wave] = l; }
  }
  __syncthreads();
  // workgroup partial: merge the 4 waves
  const int64_t chunks = gridDim.y;
  float* dst = a.partial + (row * chunks + blockIdx.y) * (DP + 2);
  float mm = fmaxf(fmaxf(part_m[0], part_m[1]), fmaxf(part_m[2], part_m[3]));
  float w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = mm == kNegInf ? 0.f : fast_exp2(part_m[i] - mm);
  for (int d = threadIdx.x; d < DP; d += 256)
    dst[2 + d] = w[0] * part_o[0][d] + w[1] * part_o[1][d] + w[2] * part_o[2][d] + w[3] * part_o[3][d];
  if (threadIdx.x == 0) {
    dst[0] = mm;
    dst[1] = w[0] * part_l[0] + w[1] * part_l[1] + w[2] * part_l[2] + w[3] * part_l[3];
  }
}

// One wave per row. The slot partials were written just before, so the
// kernel is bound by load latency: each lane fetches one chunk's (max, mass)
// and the chunk outputs are read eight chunks at a time, all loads of a
// round in flight together.
template <typename T, int DP, typename TO = T>
__global__ __launch_bounds__(64) void sparse_merge_kernel(SparseArgs a, int chunks) {
  constexpr int S = DP + 2;
  constexpr int NJ = DP / 64;
  constexpr int R = 8;
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;
  const float* src = a.partial + row * chunks * S;
  float mm = kNegInf;
  for (int c = lane; c < chunks; c += 64) mm = fmaxf(mm, src[(int64_t)c * S]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mm = fmaxf(mm, __shfl_xor(mm, off, 64));
  float l = 0.f;
  float o[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) o[j] = 0.f;
  for (int c0 = 0; c0 < chunks; c0 += 64) {
    const int c = c0 + lane;
    float w = 0.f;
    if (c < chunks && mm != kNegInf) {
      const float* pc = src + (int64_t)c * S;
      w = fast_exp2(pc[0] - mm);
      l += w * pc[1];
    }
    const int n = chunks - c0 < 64 ? chunks - c0 : 64;
    for (int i0 = 0; i0 < n; i0 += R) {
      float v[R][NJ];
#pragma unroll
      for (int i = 0; i < R; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          v[i][j] = i0 + i < n ? src[(int64_t)(c0 + i0 + i) * S + 2 + lane + 64 * j] : 0.f;
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const float wi = __shfl(w, i0 + i, 64);
#pragma unroll
        for (int j = 0; j < NJ; ++j) o[j] += wi * v[i][j];
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off, 64);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  TO* out = reinterpret_cast<TO*>(a.out) + row * a.D;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int d = lane + 64 * j;
    if (d < a.D) out[d] = from_float<TO>(o[j] * inv);
  }
  if (a.lse && lane == 0) a.lse[row] = (l > 0.f && mm != kNegInf) ? (mm + fast_log2(l)) * kLn2 : kNegInf;
}

// ---------------------------------------------------------------------------
template <typename T, int DP>
static hipError_t scores_dp(const SparseArgs& a, hipStream_t s) {
  auto note_scores = [&](const void* f, const char* name, dim3 g) {
    note_launch(f, {name, dtype_code<T>(), DP, a.block, 128, 16, 4, 1, g.x * g.y * g.z,
                    a.kv.page_table ? "paged" : "contiguous"});
  };
  const int64_t chunks = (a.kv.n_tokens + 127) / 128;
  dim3 grid((unsigned)((chunks + 3) / 4), a.H, a.B);
  if constexpr (sizeof(T) == 2 && DP <= 128) {
    if (a.D % 8 != 0) {
      // rows that are not 16-byte multiples: the element-load kernel
      note_scores((const void*)&sparse_scores_kernel<T, DP, true>, "sparse_scores", grid);
      if (a.kv.page_table) hipLaunchKernelGGL((sparse_scores_kernel<T, DP, true>), grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((sparse_scores_kernel<T, DP, false>), grid, dim3(256), 0, s, a);
      return hipGetLastError();
    }
    if (a.D % 32 == 0) {
      if ((chunks + 3) / 4 * a.H >= (int64_t(1) << 31)) return hipErrorInvalidConfiguration;
      grid = dim3((unsigned)((chunks + 3) / 4 * a.H), 1, a.B);
      auto go16 = [&]<int LOGB>() {
        note_scores((const void*)&sparse_scan16_kernel<T, DP, true, LOGB>, "sparse_scan16", grid);
        if (a.kv.page_table) hipLaunchKernelGGL((sparse_scan16_kernel<T, DP, true, LOGB>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((sparse_scan16_kernel<T, DP, false, LOGB>), grid, dim3(256), 0, s, a);
      };
      switch (a.logb) {
        case 1: go16.template operator()<1>(); break;
        case 2: go16.template operator()<2>(); break;
        case 3: go16.template operator()<3>(); break;
        case 4: go16.template operator()<4>(); break;
        case 5: go16.template operator()<5>(); break;
        case 6: go16.template operator()<6>(); break;
        default: go16.template operator()<7>(); break;
      }
      return hipGetLastError();
    }
    dim3 g1((unsigned)chunks, a.H, a.B);
    auto go = [&]<int LOGB>() {
      note_scores((const void*)&sparse_scan_kernel<T, DP, true, LOGB>, "sparse_scan", g1);
      if (a.kv.page_table) hipLaunchKernelGGL((sparse_scan_kernel<T, DP, true, LOGB>), g1, dim3(64), 0, s, a);
      else hipLaunchKernelGGL((sparse_scan_kernel<T, DP, false, LOGB>), g1, dim3(64), 0, s, a);
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
  } else {
    note_scores((const void*)&sparse_scores_kernel<T, DP, true>, "sparse_scores", grid);
    if (a.kv.page_table) hipLaunchKernelGGL((sparse_scores_kernel<T, DP, true>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((sparse_scores_kernel<T, DP, false>), grid, dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t scores_t(const SparseArgs& a, hipStream_t s) {
  if (a.D <= 64) return scores_dp<T, 64>(a, s);
  if (a.D <= 128) return scores_dp<T, 128>(a, s);
  return scores_dp<T, 256>(a, s);
}

hipError_t launch_sparse_scores(int dtype, const SparseArgs& a, hipStream_t stream) {
  switch (dtype) {
    case 2: return scores_t<bf16>(a, stream);
    case 1: return scores_t<f16>(a, stream);
    default: return scores_t<float>(a, stream);
  }
}

hipError_t launch_sparse_select(int64_t rows, int64_t n_blocks, int topk, int64_t id_base,
                                const float* scores, int64_t* ids, float* top, float* log_zr,
                                hipStream_t stream) {
  auto note = [&](const void* f, const char* name, int threads) {
    note_launch(f, {name, 0, 0, 0, 1, (int)(n_blocks < 0x7fffffff ? n_blocks : 0x7fffffff), threads / 64, 0,
                    (unsigned)rows, "row"});
  };
  if (topk <= 64 && n_blocks <= 512 * 16) note((const void*)&sparse_select_radix_kernel<512, 16>, "sparse_select_radix", 512);
  else if (topk <= 64 && n_blocks <= 512 * 32) note((const void*)&sparse_select_radix_kernel<512, 32>, "sparse_select_radix", 512);
  else if (topk <= 64) note((const void*)&sparse_select64_kernel, "sparse_select64", 256);
  else note((const void*)&sparse_select_kernel, "sparse_select", 256);
  if (topk <= 64 && n_blocks <= 512 * 16)
    hipLaunchKernelGGL((sparse_select_radix_kernel<512, 16>), dim3((unsigned)rows), dim3(512), 0, stream, n_blocks,
                       topk, id_base, scores, ids, top, log_zr);
  else if (topk <= 64 && n_blocks <= 512 * 32)
    hipLaunchKernelGGL((sparse_select_radix_kernel<512, 32>), dim3((unsigned)rows), dim3(512), 0, stream, n_blocks,
                       topk, id_base, scores, ids, top, log_zr);
  else if (topk <= 64)
    hipLaunchKernelGGL(sparse_select64_kernel, dim3((unsigned)rows), dim3(256), 0, stream, n_blocks, topk, id_base,
                       scores, ids, top, log_zr);
  else
    hipLaunchKernelGGL(sparse_select_kernel, dim3((unsigned)rows), dim3(256), 0, stream, n_blocks, topk, id_base,
                       scores, ids, top, log_zr);
  return hipGetLastError();
}

template <typename T, int DP>
static hipError_t pop_dp(const SparseArgs& a, hipStream_t s) {
  const int64_t rows = (int64_t)a.B * a.Q * a.H;
  const int chunks = (int)sparse_chunks(a.topk);
  dim3 grid((unsigned)rows, chunks);
  note_launch((const void*)&sparse_pop_kernel<T, DP, true>,
              {"sparse_pop", dtype_code<T>(), DP, a.block, 1, a.block, 4, 0, grid.x * grid.y,
               a.kv.page_table ? "paged" : "contiguous"});
  note_launch((const void*)&sparse_merge_kernel<T, DP>,
              {"sparse_merge", dtype_code<T>(), DP, a.block, 1, DP, 1, 0, grid.x, "row"});
  if (a.kv.page_table) hipLaunchKernelGGL((sparse_pop_kernel<T, DP, true>), grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((sparse_pop_kernel<T, DP, false>), grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (a.out_f32) hipLaunchKernelGGL((sparse_merge_kernel<T, DP, float>), dim3((unsigned)rows), dim3(64), 0, s, a, chunks);
  else hipLaunchKernelGGL((sparse_merge_kernel<T, DP>), dim3((unsigned)rows), dim3(64), 0, s, a, chunks);
  return hipGetLastError();
}

template <typename T>
static hipError_t pop_t(const SparseArgs& a, hipStream_t s) {
  if (a.D <= 64) return pop_dp<T, 64>(a, s);
  if (a.D <= 128) return pop_dp<T, 128>(a, s);
  return pop_dp<T, 256>(a, s);
}

hipError_t launch_sparse_pop(int dtype, const SparseArgs& a, hipStream_t stream) {
  switch (dtype) {
    case 2: return pop_t<bf16>(a, stream);
    case 1: return pop_t<f16>(a, stream);
    default: return pop_t<float>(a, stream);
  }
}

}  // namespace st
