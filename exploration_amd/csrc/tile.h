// Tile building blocks shared by the dense forward and backward kernels:
// LDS staging of key/value tiles, MFMA products in the transposed layout and
// per-(row, key block) reductions.
#pragma once

#include <utility>

#include "common.h"

namespace st {

// LDS row strides (elements). Row-major tiles pad 16 bytes per row;
// transposed 16-bit tiles pad 8 bytes so that 32 lanes reading 8 bytes from
// 32 consecutive rows hit distinct banks.
template <typename T, int DP> struct RowLd { static constexpr int value = DP + 16 / (int)sizeof(T); };
template <int NT> struct TLd { static constexpr int value = NT + 4; };

template <typename T> struct Vec16;
template <> struct Vec16<bf16> { typedef bf16x8 type; static constexpr int n = 8; };
template <> struct Vec16<f16> { typedef f16x8 type; static constexpr int n = 8; };
template <> struct Vec16<float> { typedef f32x4 type; static constexpr int n = 4; };

// Copy rows [r0, r0+ROWS) x columns [0, DP) of a [*, stride] matrix into LDS
// (row-major, stride LD), zero-filling rows >= nrows and columns >= ncols.
// ncols must be a multiple of 16 bytes worth of elements.
template <typename T, int ROWS, int DP, int LD, int NTHREADS>
__device__ __forceinline__ void stage_rows(T* lds, const T* g, int64_t stride, int r0, int nrows,
                                           int ncols) {
  typedef typename Vec16<T>::type V;
  constexpr int E = Vec16<T>::n;
  constexpr int CPR = DP / E;
  constexpr int TOTAL = ROWS * CPR;
#pragma unroll
  for (int it = 0; it < (TOTAL + NTHREADS - 1) / NTHREADS; ++it) {
    const int id = threadIdx.x + it * NTHREADS;
    if (TOTAL % NTHREADS != 0 && id >= TOTAL) break;
    const int n = id / CPR, c = (id % CPR) * E;
    V val = {};
    if (r0 + n < nrows && c < ncols) val = load_vec<V>(g + (int64_t)(r0 + n) * stride + c);
    *reinterpret_cast<V*>(lds + n * LD + c) = val;
  }
}

// Same source, stored transposed: lds[c][n] (stride LDT) for 16-bit types.
template <typename T, int ROWS, int DP, int LDT, int NTHREADS>
__device__ __forceinline__ void stage_rows_t(T* lds, const T* g, int64_t stride, int r0, int nrows,
                                             int ncols) {
  typedef typename Vec16<T>::type V;
  constexpr int E = Vec16<T>::n;
  constexpr int CPR = DP / E;
  constexpr int TOTAL = ROWS * CPR;
#pragma unroll
  for (int it = 0; it < (TOTAL + NTHREADS - 1) / NTHREADS; ++it) {
    const int id = threadIdx.x + it * NTHREADS;
    if (TOTAL % NTHREADS != 0 && id >= TOTAL) break;
    const int n = id % ROWS, c = (id / ROWS) * E;
    V val = {};
    if (r0 + n < nrows && c < ncols) val = load_vec<V>(g + (int64_t)(r0 + n) * stride + c);
#pragma unroll
    for (int e = 0; e < E; ++e) lds[(c + e) * LDT + n] = val[e];
  }
}

// Operand fragment for row `row` of a row-major LDS tile, contraction chunk c:
// elements [c*KW + half*VEC, +VEC).
template <typename T, int LD>
__device__ __forceinline__ typename Mma<T>::Frag frag_row(const T* lds, int row, int c, int half) {
  typedef typename Mma<T>::Frag F;
  return *reinterpret_cast<const F*>(lds + row * LD + c * Mma<T>::KW + half * Mma<T>::VEC);
}

// Operand fragment from a transposed 16-bit LDS tile (lds[r][key]) for row r
// and the 16 keys [k0, k0+16) in the permuted order that matches the C-tile
// layout: slots 0..3 <-> k0+4h+{0..3}, slots 4..7 <-> k0+8+4h+{0..3}.
template <typename T, int LDT>
__device__ __forceinline__ typename Mma<T>::Frag frag_t16(const T* lds, int r, int k0, int half) {
  typedef T V4 __attribute__((ext_vector_type(4)));
  const T* p = lds + r * LDT + k0 + 4 * half;
  V4 lo = *reinterpret_cast<const V4*>(p);
  V4 hi = *reinterpret_cast<const V4*>(p + 8);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// B-operand fragment (16-bit) from C-tile registers [8*c2, 8*c2+8) of x.
template <typename T>
__device__ __forceinline__ typename Mma<T>::Frag frag_from_c(const f32x16& x, int c2) {
  typename Mma<T>::Frag f;
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = from_float<T>(x[8 * c2 + e]);
  return f;
}

// S^T tile (NT keys x 32 rows) = K_tile . Q^T with K staged row-major in LDS
// (stride LDK) and Q^T held in registers as fragments qf[DP/KW].
template <typename T, int NST, int NKC, int LDK>
__device__ __forceinline__ void scores_t(f32x16 (&s)[NST], const T* lds_k,
                                         const typename Mma<T>::Frag (&qf)[NKC], int col, int half) {
#pragma unroll
  for (int st = 0; st < NST; ++st) {
    f32x16 acc = zero16();
#pragma unroll
    for (int c = 0; c < NKC; ++c) acc = Mma<T>::mma(frag_row<T, LDK>(lds_k, 32 * st + col, c, half), qf[c], acc);
    s[st] = acc;
  }
}

// acc^T[d][row] += X^T . P^T where P is given as C tiles p[NST] (keys x rows)
// and X (values or keys) is staged in LDS: transposed [DP][LDT] for 16-bit
// types, row-major [NT][LD] for fp32.
template <typename T, int NST, int NDT, int LDX>
__device__ __forceinline__ void accumulate_t(f32x16 (&acc)[NDT], const f32x16 (&p)[NST], const T* lds_x,
                                             int col, int half) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int st = 0; st < NST; ++st) {
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        const typename Mma<T>::Frag b = frag_from_c<T>(p[st], c2);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
          acc[dt] = Mma<T>::mma(frag_t16<T, LDX>(lds_x, 32 * dt + col, 32 * st + 16 * c2, half), b, acc[dt]);
      }
    }
  } else {
#pragma unroll
    for (int st = 0; st < NST; ++st) {
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int key = 32 * st + c_row(t, half);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
          acc[dt] = Mma<T>::mma(lds_x[key * LDX + 32 * dt + col], p[st][t], acc[dt]);
      }
    }
  }
}

// Per-(row, key block) sums of x over the keys of each block, for a tile of
// NST C tiles with block size 2^LOGB (the tile holds whole blocks). blk[st][j]
// receives the sum of block slot j of subtile st; blk_slot maps a register
// to its slot. For LOGB >= 5 every subtile of a block gets the block total.
template <int LOGB> __device__ __forceinline__ constexpr int blk_slot(int r) {
  return LOGB == 1 ? (r >> 1) : (LOGB <= 3 ? (r >> 2) : (LOGB == 4 ? (r >> 3) : 0));
}

struct OpAdd {
  static __device__ __forceinline__ float f(float x, float y) { return x + y; }
  static __device__ __forceinline__ float other(float x) { return other_half(x); }
};
struct OpMax {
  static __device__ __forceinline__ float f(float x, float y) { return fmaxf(x, y); }
  static __device__ __forceinline__ float other(float x) { return other_half(x); }
};

// Op over the 16 registers of a C tile as a balanced tree.
template <typename Op> __device__ __forceinline__ float tree16(const f32x16& x) {
  float a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = Op::f(x[2 * i], x[2 * i + 1]);
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = Op::f(a[2 * i], a[2 * i + 1]);
  return Op::f(Op::f(a[0], a[1]), Op::f(a[2], a[3]));
}

template <int NST, int LOGB, typename Op = OpAdd>
__device__ __forceinline__ void block_sums(const f32x16 (&x)[NST], float (&blk)[NST][8]) {
  if constexpr ((1 << LOGB) > 32 * NST) {
    // block larger than the tile: never dispatched (tiles hold whole blocks)
  } else if constexpr (LOGB >= 5) {
    constexpr int G = (1 << LOGB) / 32;  // subtiles per block
    float t[NST];
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      float acc = x[st][0];
#pragma unroll
      for (int r = 1; r < 16; ++r) acc = Op::f(acc, x[st][r]);
      t[st] = acc;
    }
#pragma unroll
    for (int st = 0; st < NST; ++st) t[st] = Op::f(t[st], Op::other(t[st]));
#pragma unroll
    for (int g0 = 0; g0 < NST; g0 += G) {
      float tot = t[g0];
#pragma unroll
      for (int g = 1; g < G; ++g) tot = Op::f(tot, t[g0 + g]);
#pragma unroll
      for (int g = 0; g < G; ++g) blk[g0 + g][0] = tot;
    }
  } else if constexpr (LOGB == 4) {
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      float a0 = x[st][0], a1 = x[st][8];
#pragma unroll
      for (int r = 1; r < 8; ++r) { a0 = Op::f(a0, x[st][r]); a1 = Op::f(a1, x[st][r + 8]); }
      blk[st][0] = Op::f(a0, Op::other(a0));
      blk[st][1] = Op::f(a1, Op::other(a1));
    }
  } else if constexpr (LOGB == 3) {
#pragma unroll
    for (int st = 0; st < NST; ++st) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a = Op::f(Op::f(x[st][4 * i], x[st][4 * i + 1]), Op::f(x[st][4 * i + 2], x[st][4 * i + 3]));
        blk[st][i] = Op::f(a, Op::other(a));
      }
    }
  } else if constexpr (LOGB == 2) {
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        blk[st][i] = Op::f(Op::f(x[st][4 * i], x[st][4 * i + 1]), Op::f(x[st][4 * i + 2], x[st][4 * i + 3]));
  } else {
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int i = 0; i < 8; ++i) blk[st][i] = Op::f(x[st][2 * i], x[st][2 * i + 1]);
  }
}

// block_sums in two parts, so that the in-lane part of one subtile can run
// beside the MFMAs of the next. block_part: this lane's slot sums of one C
// tile (of x, or with DOT of x*y as a chain of FMAs, one instruction per
// element); block_finish: the other half-wave's part (blocks of 8+ keys)
// and, for blocks of several subtiles, their total.
template <int LOGB, bool DOT>
__device__ __forceinline__ void block_part(const f32x16& x, const f32x16& y, float (&part)[8]) {
  auto first = [&](int r) { return DOT ? x[r] * y[r] : x[r]; };
  auto next = [&](float a, int r) { return DOT ? fmaf(x[r], y[r], a) : a + x[r]; };
  if constexpr (LOGB >= 5) {
    float a = first(0);
#pragma unroll
    for (int r = 1; r < 16; ++r) a = next(a, r);
    part[0] = a;
  } else if constexpr (LOGB == 4) {
    float a0 = first(0), a1 = first(8);
#pragma unroll
    for (int r = 1; r < 8; ++r) { a0 = next(a0, r); a1 = next(a1, r + 8); }
    part[0] = a0;
    part[1] = a1;
  } else if constexpr (LOGB >= 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float a = first(4 * i);
#pragma unroll
      for (int e = 1; e < 4; ++e) a = next(a, 4 * i + e);
      part[i] = a;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) part[i] = next(first(2 * i), 2 * i + 1);
  }
}

template <int NST, int LOGB>
__device__ __forceinline__ void block_finish(const float (&part)[NST][8], float (&blk)[NST][8]) {
  if constexpr ((1 << LOGB) > 32 * NST) {
    // block larger than the tile: never dispatched (tiles hold whole blocks)
  } else if constexpr (LOGB >= 5) {
    constexpr int G = (1 << LOGB) / 32;  // subtiles per block
    float t[NST];
#pragma unroll
    for (int st = 0; st < NST; ++st) t[st] = part[st][0] + other_half(part[st][0]);
#pragma unroll
    for (int g0 = 0; g0 < NST; g0 += G) {
      float tot = t[g0];
#pragma unroll
      for (int g = 1; g < G; ++g) tot += t[g0 + g];
#pragma unroll
      for (int g = 0; g < G; ++g) blk[g0 + g][0] = tot;
    }
  } else {
    constexpr int NSL = LOGB == 4 ? 2 : (LOGB >= 2 ? 4 : 8);  // slots per subtile
#pragma unroll
    for (int st = 0; st < NST; ++st)
#pragma unroll
      for (int j = 0; j < NSL; ++j) blk[st][j] = LOGB >= 3 ? part[st][j] + other_half(part[st][j]) : part[st][j];
  }
}

// Index, within the tile, of the key block that slot j of subtile st in a
// lane of half h refers to (block size 2^LOGB, NST subtiles of 32 keys).
template <int LOGB> __device__ __forceinline__ int blk_index(int st, int j, int h) {
  if constexpr (LOGB >= 5) return (32 * st) >> LOGB;
  else if constexpr (LOGB == 4) return 2 * st + j;
  else if constexpr (LOGB == 3) return 4 * st + j;
  else if constexpr (LOGB == 2) return 8 * st + 2 * j + h;
  else return 16 * st + 4 * (j >> 1) + 2 * h + (j & 1);
}
// Slots per subtile that carry distinct blocks, and whether the two halves of
// the wave hold different blocks (block size <= 4).
template <int LOGB> struct BlkSlots {
  static constexpr int n = LOGB >= 5 ? 1 : (LOGB == 4 ? 2 : (LOGB >= 2 ? 4 : 8));
  static constexpr bool per_half = LOGB <= 2;
};

// ---------------------------------------------------------------------------
// Asynchronously staged, XOR-swizzled row-major tiles (16-bit types).
// A tile row of DP elements is CPR = DP/8 chunks of 16 bytes; logical chunk c
// of row r is stored at chunk c ^ swz(r). gfx950's LDS serves a 16-lane phase
// of a ds_read_b128 or ds_read_tr16_b64 from 64 four-byte banks (256 bytes),
// and the swizzle keeps both fragment reads of the dense kernels free of bank
// conflicts (measured: 208 B/clk/CU for the b128 pattern against 126 with a
// period-8 swizzle):
//  * 16 consecutive rows read at one logical chunk (ds_read_b128 fragments,
//    lanes = rows) land in 16 distinct 16-byte slots of the 256-byte period;
//  * 4 consecutive rows read 32 logical bytes each (ds_read_tr16_b64
//    fragments) land in 4 distinct 32-byte slots.
// DP = 128 (256-byte rows): swz = 2*(r%8) + (r/8)%2. DP = 64 (128-byte rows,
// row parity already separates two halves of the period): swz = 2*b1 ^ b2 ^
// 4*b3 over bits b_k of r. The period is 16 rows for both.
template <int DP> __device__ __forceinline__ int swz(int r) {
  static_assert(DP == 64 || DP == 128, "swizzled tiles have 64 or 128 columns");
  if constexpr (DP == 128) return 2 * (r & 7) + ((r >> 3) & 1);
  else return (((r >> 1) & 1) << 1) ^ ((r >> 2) & 1) ^ (((r >> 3) & 1) << 2);
}
constexpr int kSwzPeriod = 16;  // swz(r + 16) == swz(r)

// Asynchronous copies of full-width row tiles (rows [r0, r0+ROWS) x [0, DP)
// of a [nrows, stride] matrix with DP columns) into the swizzled LDS layout.
// One instruction of the NWAVES waves moves a slab of RPI rows, and a lane's
// position within a slab (row, swizzled chunk) is the same for every slab, so
// each copy's address is the matrix base plus a 32-bit byte offset: the
// lane's fixed offset plus the slab's (32-bit arithmetic only, whether the
// compiler keeps the uniform parts in scalar or vector registers). In a slab
// that crosses row nrows the rows at or beyond it re-read row nrows-1 (finite
// data whose products are masked or discarded). Every wave of the workgroup
// takes part. The host keeps nrows * stride * sizeof(T) below 2^31.
template <typename T, int DP, int NWAVES> struct Stager {
  static_assert(sizeof(T) == 2, "16-bit tiles");
  static constexpr int CPR = DP / 8;                // 16-byte chunks per row
  static constexpr int RPI = NWAVES * 64 / CPR;     // rows per slab
  static_assert(RPI % kSwzPeriod == 0, "a slab must keep the swizzle phase");
  const char* base;
  uint32_t row_bytes;
  int nrows, r_lane, wave;
  uint32_t voff;  // r_lane * row_bytes + 16 * swizzled chunk
  // tid: this thread's index among the NWAVES * 64 threads that stage (the
  // workgroup, or one group of its waves)
  __device__ __forceinline__ Stager(const T* base_, int64_t stride, int nrows_, int tid = (int)threadIdx.x) {
    const int p = tid;
    // wave-uniform (scalar) so that the LDS destinations are scalar too
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    r_lane = p / CPR;
    const int chunk = (p % CPR) ^ swz<DP>(r_lane);
    // the matrix base in SGPRs: every copy then takes the scalar-base form
    // (SGPR pair + 32-bit VGPR offset, no 64-bit address arithmetic)
    const uint64_t b64 = reinterpret_cast<uint64_t>(base_);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b64);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b64 >> 32));
    base = reinterpret_cast<const char*>(((uint64_t)hi << 32) | lo);
    row_bytes = (uint32_t)(stride * (int64_t)sizeof(T));
    nrows = nrows_;
    voff = (uint32_t)r_lane * row_bytes + (uint32_t)chunk * 16u;
  }
  template <int ROWS>
  __device__ __forceinline__ void stage(T* lds, int r0) const {
    static_assert(ROWS % RPI == 0, "tile must split into whole slabs");
    if (r0 + ROWS <= nrows) {
      const uint32_t s0 = (uint32_t)r0 * row_bytes, slab = (uint32_t)RPI * row_bytes;
#pragma unroll
      for (int it = 0; it < ROWS / RPI; ++it)
        async_copy16(base + (voff + (s0 + (uint32_t)it * slab)), lds + (it * NWAVES + wave) * 64 * 8);
    } else {
      // recomputed per call: hoisting r_lane + it*RPI out of the caller's
      // loop would hold (or spill) one register per slab
      int rl = r_lane;
      __asm__ volatile("" : "+v"(rl));
      const uint32_t cb = voff - (uint32_t)r_lane * row_bytes;
#pragma unroll
      for (int it = 0; it < ROWS / RPI; ++it) {
        int row = r0 + it * RPI + rl;
        row = row < nrows ? row : nrows - 1;
        async_copy16(base + ((uint32_t)row * row_bytes + cb), lds + (it * NWAVES + wave) * 64 * 8);
      }
    }
  }
};

// MFMA fragment (8 elements) of swizzled row n, logical chunk c.
template <typename T, int DP>
__device__ __forceinline__ typename Mma<T>::Frag frag_swz(const T* lds, int n, int c) {
  return *reinterpret_cast<const typename Mma<T>::Frag*>(lds + n * DP + ((c ^ swz<DP>(n)) * 8));
}

// Transposed MFMA fragment from a swizzled row-major tile X[key][d]: the A
// operand of acc^T[d][row] += X^T P^T for dims [d0, d0+32) and the 16 keys
// [k0, k0+16), in the permuted key order of frag_from_c (slots 0..3 <->
// k0+4h+{0..3}, slots 4..7 <-> k0+8+4h+{0..3}). Two ds_read_tr16_b64: within
// each 16-lane group, out[i][j] = in[4j + i/4][i%4] where in[s] is the 8
// bytes lane s reads, so lane s reads row k+s/4, dims d+4(s%4)..+3.
template <typename T, int DP>
__device__ __forceinline__ typename Mma<T>::Frag frag_tr(const T* lds, int k0, int d0, int lane) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  const int gi = lane >> 4, s = lane & 15;
  const int half = gi >> 1;
  const int d = d0 + 16 * (gi & 1) + 4 * (s & 3);
  const int row0 = k0 + 4 * half + (s >> 2);
  const int row1 = row0 + 8;
  const int lc = d >> 3, off = d & 7;
  const T* p0 = lds + row0 * DP + ((lc ^ swz<DP>(row0)) * 8) + off;
  const T* p1 = lds + row1 * DP + ((lc ^ swz<DP>(row1)) * 8) + off;
  s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)p0);
  s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)p1);
  typedef short s8 __attribute__((ext_vector_type(8)));
  s8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(typename Mma<T>::Frag, v);
}

// A chain of C chunks of L MFMAs over several products (what would be
// consecutive phases), with one chunk of read-ahead throughout: the operand
// reads of chunk g+1 are issued before chunk g's MFMAs, also where the
// products change, so no phase starts with an exposed LDS latency. The wait
// is an explicit lgkmcnt(0) at each chunk boundary (with asynchronous
// global->LDS copies in flight the compiler only ever waits for all LDS
// reads, so a read issued right before its MFMA would stall it); here every
// read has a whole chunk of MFMAs to land. Product J is
// load.template operator()<J>() then mma.template operator()<J>(frag);
// after.template operator()<g>() (VALU work, which may read results of
// chunks <= g only) follows chunk g's MFMAs in the same scheduling region.
template <int C, int L, typename Load, typename Mfma, typename After>
__device__ __forceinline__ void mfma_chain(Load&& load, Mfma&& mma, After&& after) {
  typedef decltype(load.template operator()<0>()) F;
  F buf[2][L];
  [&]<int... I>(std::integer_sequence<int, I...>) {
    ((buf[0][I] = load.template operator()<I>()), ...);
  }(std::make_integer_sequence<int, L>{});
  [&]<int... G>(std::integer_sequence<int, G...>) {
    ([&] {
      constexpr int g = G;
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt untouched
      __builtin_amdgcn_sched_barrier(0);
      [&]<int... I>(std::integer_sequence<int, I...>) {
        if constexpr (g + 1 < C) ((buf[(g + 1) & 1][I] = load.template operator()<(g + 1) * L + I>()), ...);
        (mma.template operator()<g * L + I>(buf[g & 1][I]), ...);
      }(std::make_integer_sequence<int, L>{});
      after.template operator()<g>();
    }(), ...);
  }(std::make_integer_sequence<int, C>{});
  __builtin_amdgcn_sched_barrier(0);
}

// ---------------------------------------------------------------------------
// 16x16x32 MFMA layout helpers (v_mfma_f32_16x16x32_{bf16,f16}): a C tile
// of S^T = K Q^T puts query row l%16 in lane l and keys 4*(l/16)+r
// (r = 0..3) of a 16-key subtile in its registers, so a row's values are
// spread over the four 16-lane rows of the wave (lanes i, i+16, i+32, i+48).

// Op over lanes i and i^16 (16-lane rows 0/1 and 2/3), result in both: one
// v_permlane16_swap returns the pair's two values in its two outputs.
template <typename Op> __device__ __forceinline__ float reduce_pair16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return Op::f(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Op over lanes i and i^32.
template <typename Op> __device__ __forceinline__ float reduce_pair32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return Op::f(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Op over the four 16-lane rows (a query row's lanes), result in all four.
template <typename Op> __device__ __forceinline__ float reduce_rows4(float x) {
  return reduce_pair32<Op>(reduce_pair16<Op>(x));
}

template <typename Op> __device__ __forceinline__ float op4(const f32x4& x) {
  return Op::f(Op::f(x[0], x[1]), Op::f(x[2], x[3]));
}

// Per-(row, key block) reductions of NSUB 16-key C subtiles (block size
// 2^LOGB, the subtiles hold whole blocks). blk[t][s] receives the total of
// block slot s of subtile t in every lane that holds part of the block:
// block size 2 has two slots per subtile (registers 0-1, 2-3), larger sizes
// one. Blocks of 32..128 keys span 2..8 subtiles; each of them gets the
// block total.
template <int LOGB> __device__ __forceinline__ constexpr int slot16(int r) { return LOGB == 1 ? (r >> 1) : 0; }
template <int LOGB> struct Slots16 { static constexpr int n = LOGB == 1 ? 2 : 1; };

template <int NSUB, int LOGB, typename Op = OpAdd>
__device__ __forceinline__ void block_sums16(const f32x4 (&x)[NSUB], float (&blk)[NSUB][2]) {
  if constexpr (LOGB == 1) {
#pragma unroll
    for (int t = 0; t < NSUB; ++t) {
      blk[t][0] = Op::f(x[t][0], x[t][1]);
      blk[t][1] = Op::f(x[t][2], x[t][3]);
    }
  } else if constexpr (LOGB == 2) {
#pragma unroll
    for (int t = 0; t < NSUB; ++t) blk[t][0] = op4<Op>(x[t]);
  } else if constexpr (LOGB == 3) {
#pragma unroll
    for (int t = 0; t < NSUB; ++t) blk[t][0] = reduce_pair16<Op>(op4<Op>(x[t]));
  } else if constexpr (LOGB == 4) {
#pragma unroll
    for (int t = 0; t < NSUB; ++t) blk[t][0] = reduce_rows4<Op>(op4<Op>(x[t]));
  } else {
    constexpr int G = (1 << LOGB) / 16 < NSUB ? (1 << LOGB) / 16 : NSUB;
#pragma unroll
    for (int t0 = 0; t0 < NSUB; t0 += G) {
      float tot = op4<Op>(x[t0]);
#pragma unroll
      for (int t = t0 + 1; t < t0 + G; ++t) tot = Op::f(tot, op4<Op>(x[t]));
      tot = reduce_rows4<Op>(tot);
#pragma unroll
      for (int t = t0; t < t0 + G; ++t) blk[t][0] = tot;
    }
  }
}

// block_sums16 for blocks of 4+ keys from the subtiles' in-lane partials
// part[t] (the op over the lane's four values of subtile t).
template <int NSUB, int LOGB, typename Op = OpAdd>
__device__ __forceinline__ void block_sums16_from(const float (&part)[NSUB], float (&blk)[NSUB][2]) {
  static_assert(LOGB >= 2, "blocks of 2 keys need the single values");
  if constexpr (LOGB == 2) {
#pragma unroll
    for (int t = 0; t < NSUB; ++t) blk[t][0] = part[t];
  } else if constexpr (LOGB == 3) {
#pragma unroll
    for (int t = 0; t < NSUB; ++t) blk[t][0] = reduce_pair16<Op>(part[t]);
  } else if constexpr (LOGB == 4) {
#pragma unroll
    for (int t = 0; t < NSUB; ++t) blk[t][0] = reduce_rows4<Op>(part[t]);
  } else {
    constexpr int G = (1 << LOGB) / 16 < NSUB ? (1 << LOGB) / 16 : NSUB;
#pragma unroll
    for (int t0 = 0; t0 < NSUB; t0 += G) {
      float tot = part[t0];
#pragma unroll
      for (int t = t0 + 1; t < t0 + G; ++t) tot = Op::f(tot, part[t]);
      tot = reduce_rows4<Op>(tot);
#pragma unroll
      for (int t = t0; t < t0 + G; ++t) blk[t][0] = tot;
    }
  }
}

// Whether block slot s of subtile t counts in a lane of 16-lane row g when
// a per-row sum over blocks is later reduced over the four rows (each block
// once).
template <int LOGB> __device__ __forceinline__ bool owns16(int t, int g) {
  if constexpr (LOGB <= 2) return true;
  else if constexpr (LOGB == 3) return (g & 1) == 0;
  else if constexpr (LOGB == 4) return g == 0;
  else return g == 0 && (t % ((1 << LOGB) / 16)) == 0;
}

// An MFMA phase of N products in chunks of L whose A operands are read from
// LDS (the first NR2 products two reads each, e.g. transposed V fragments,
// the rest one), read one chunk ahead as in mfma_chain; the chunks from NQ0
// on also read one fragment shared by their L products (the B operand of
// the S^T products, one Q fragment per contraction chunk), with the chunk's
// own operands, and hand it to mma(j, f, shared) (chunks before NQ0 get an
// unused fragment).
template <int N, int L, int NR2, int NQ0, typename Load, typename QLoad, typename Mfma>
__device__ __forceinline__ void mfma_chunks_shared(Load&& load, QLoad&& qload, Mfma&& mma) {
  static_assert(N % L == 0 && NR2 % L == 0 && NQ0 % L == 0, "phase must split into whole chunks");
  constexpr int C = N / L;
  typedef decltype(load(0)) F;
  F buf[2][L];
  F qb[2];
#pragma unroll
  for (int i = 0; i < L; ++i) buf[0][i] = load(i);
  if constexpr (NQ0 == 0) qb[0] = qload(0);
  [&]<int... G>(std::integer_sequence<int, G...>) {
    ([&] {
      constexpr int g = G;
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt untouched
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (g + 1 < C) {
#pragma unroll
        for (int i = 0; i < L; ++i) buf[(g + 1) & 1][i] = load((g + 1) * L + i);
        if constexpr ((g + 1) * L >= NQ0) qb[(g + 1) & 1] = qload(g + 1);
      }
#pragma unroll
      for (int i = 0; i < L; ++i) mma(g * L + i, buf[g & 1][i], qb[g & 1]);
      if constexpr (g + 1 < C)
        __builtin_amdgcn_sched_group_barrier(
            0x100, L * ((g + 1) * L < NR2 ? 2 : 1) + ((g + 1) * L >= NQ0 ? 1 : 0), 0);
      __builtin_amdgcn_sched_group_barrier(0x008, L, 0);
    }(), ...);
  }(std::make_integer_sequence<int, C>{});
  __builtin_amdgcn_sched_barrier(0);
}

// Half-wave exchange: returns x of the lane 32 positions away.
__device__ __forceinline__ float swap_halves(float x) { return other_half(x); }

// Runs body.template operator()<LOGB>() for the runtime block size.
template <typename F> __device__ __forceinline__ void dispatch_logb(int logb, F&& body) {
  switch (logb) {
    case 1: body.template operator()<1>(); break;
    case 2: body.template operator()<2>(); break;
    case 3: body.template operator()<3>(); break;
    case 4: body.template operator()<4>(); break;
    case 5: body.template operator()<5>(); break;
    case 6: body.template operator()<6>(); break;
    default: body.template operator()<7>(); break;
  }
}

}  // namespace st
