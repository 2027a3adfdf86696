// Multi-scale deformable attention (MSDA) for AMD Instinct MI355X (gfx950):
// forward and zero-buffer backward behind the C ABI of include/deformops_amd.h.
//
// Sample-parallel kernels (the forward, and the location / weight gradients of the
// backward). A "unit" is one (batch, query, head): it owns the D channels of one
// output vector and L * P samples. A unit is served by LH = 2^k lanes of a wave64,
// each lane holding CV consecutive channels (CV * element size <= 16 bytes, so one
// corner fetch is one global_load_dwordx4 for bf16/f16 D = 32). A wave therefore
// serves UW = 64 / LH units; a workgroup is 1-4 waves. Workgroups are renumbered so
// that consecutive units land on the same XCD (gfx950 deals workgroups to its 8
// XCDs round-robin, and each XCD has its own L2): queries that are neighbours in
// the flattened pyramid sample neighbouring pixels, so their corner gathers share
// one L2. Each such kernel runs in phases:
//   1. Every lane of a unit takes samples s = t, t + LH, ... (t = lane in unit),
//      reads its location and weight, and stages the sample's four corner byte
//      offsets and four (bilinear * attention) weights in LDS. The softmax over the
//      L * P weights of a unit is a cross-lane max / sum inside the unit's lanes.
//   2. The unit's lanes walk all L * P samples: one broadcast LDS read of the
//      staged sample, four vector corner loads, fp32 (fp64 for double) FMAs. The
//      backward forms the four per-corner dot products
//      G_c = sum_d grad_out[d] * value_c[d] instead and reduces them across the
//      unit's lanes.
//   3. (backward) The lane that staged sample s turns its G_c into the location
//      and weight gradients:
//        dL/dw   = sum_c bilinear_c * G_c
//        dL/dx   = a * W * ((1 - dy) (G01 - G00) + dy (G11 - G10))
//        dL/dy   = a * H * ((1 - dx) (G10 - G00) + dx (G11 - G01))
//      and, for the softmax method, dL/dlogit_j = p_j (dL/dp_j - sum_i p_i dL/dp_i).
// grad_value is owner-computed by tile kernels instead; see the backward section.
//
// Semantics follow the reference eager backend
// (sources/deformops/backends/eager/msda_pytorch.py:23-112): pixel = loc * size -
// 0.5 computed without FMA contraction, floor, per-corner two-sided masks, clamped
// gathers. A sample outside -1 <= pixel < size (NaN included) is skipped, as in
// include/msda_forward.cuh:100-103 of the reference CUDA kernel, so it contributes
// zero and gets zero gradients; the softmax still counts it
// (include/msda_forward.cuh:92-99).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <stdlib.h>
#include <type_traits>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "deformops_amd.h"

namespace {

constexpr int kWave = 64;
constexpr int kXcds = 8;               // gfx950: 8 XCDs, 32 CUs each
constexpr int kMaxWavesPerBlock = 4;
constexpr size_t kMaxLds = 64 * 1024;  // bytes of LDS one workgroup may take

// ---------------------------------------------------------------------------
// Element types.

struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

template <typename T> struct Elem;
template <> struct Elem<float> { using acc = float; static constexpr int size = 4; };
template <> struct Elem<double> { using acc = double; static constexpr int size = 8; };
template <> struct Elem<bf16_t> { using acc = float; static constexpr int size = 2; };
template <> struct Elem<f16_t> { using acc = float; static constexpr int size = 2; };

typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2_v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_v __attribute__((ext_vector_type(4)));

__device__ inline float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ inline float f16_bits(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}
__device__ inline uint32_t pack_bf16(float a, float b) {
  const bf16x2_v v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ inline uint32_t pack_f16(float a, float b) {
  const f16x2_v v = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// One element, widened to the accumulation type.
__device__ inline float load_acc(const float* p) { return *p; }
__device__ inline double load_acc(const double* p) { return *p; }
__device__ inline float load_acc(const bf16_t* p) { return __uint_as_float(uint32_t(p->bits) << 16); }
__device__ inline float load_acc(const f16_t* p) { return f16_bits(p->bits); }

// One element, rounded to nearest even from the accumulation type.
__device__ inline void store_elem(float* p, float v) { *p = v; }
__device__ inline void store_elem(double* p, double v) { *p = v; }
__device__ inline void store_elem(bf16_t* p, float v) {
  p->bits = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
}
__device__ inline void store_elem(f16_t* p, float v) {
  p->bits = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// CV consecutive channels of one head vector: a single 2/4/8/16-byte access.
template <int BYTES> struct alignas(BYTES) Raw { uint32_t w[BYTES / 4]; };
template <> struct alignas(2) Raw<2> { uint16_t h; };

template <typename T, int CV> struct Chan;

template <int CV> struct Chan<float, CV> {
  using R = Raw<4 * CV>;
  static __device__ inline void from_raw(const R& r, float (&v)[CV]) {
#pragma unroll
    for (int i = 0; i < CV; ++i) v[i] = __uint_as_float(r.w[i]);
  }
  static __device__ inline void load(const char* p, float (&v)[CV]) {
    from_raw(*reinterpret_cast<const R*>(p), v);
  }
  // acc + sum_i a[i] * b[i] over the CV channels.
  static __device__ inline float dot(const R& a, const R& b, float acc) {
#pragma unroll
    for (int i = 0; i < CV; ++i) acc = fma(__uint_as_float(a.w[i]), __uint_as_float(b.w[i]), acc);
    return acc;
  }
  static __device__ inline void store(char* p, const float (&v)[CV]) {
    R r;
#pragma unroll
    for (int i = 0; i < CV; ++i) r.w[i] = __float_as_uint(v[i]);
    *reinterpret_cast<R*>(p) = r;
  }
};

template <int CV> struct Chan<double, CV> {
  using R = Raw<8 * CV>;
  static __device__ inline void from_raw(const R& r, double (&v)[CV]) {
#pragma unroll
    for (int i = 0; i < CV; ++i)
      v[i] = __builtin_bit_cast(double, (uint64_t(r.w[2 * i + 1]) << 32) | r.w[2 * i]);
  }
  static __device__ inline void load(const char* p, double (&v)[CV]) {
    from_raw(*reinterpret_cast<const R*>(p), v);
  }
  static __device__ inline double dot(const R& a, const R& b, double acc) {
    double x[CV], y[CV];
    from_raw(a, x);
    from_raw(b, y);
#pragma unroll
    for (int i = 0; i < CV; ++i) acc = fma(x[i], y[i], acc);
    return acc;
  }
  static __device__ inline void store(char* p, const double (&v)[CV]) {
    R r;
#pragma unroll
    for (int i = 0; i < CV; ++i) {
      const uint64_t u = __builtin_bit_cast(uint64_t, v[i]);
      r.w[2 * i] = uint32_t(u);
      r.w[2 * i + 1] = uint32_t(u >> 32);
    }
    *reinterpret_cast<R*>(p) = r;
  }
};

// bf16 and f16 share the packing; only the conversions differ.
template <typename T, int CV> struct Chan16 {
  static constexpr bool kBf16 = sizeof(T) == 2 && __is_same(T, bf16_t);
  using R = Raw<2 * CV>;
  static __device__ inline float lo(uint32_t w) { return kBf16 ? bf16_lo(w) : f16_bits(w & 0xffffu); }
  static __device__ inline float hi(uint32_t w) { return kBf16 ? bf16_hi(w) : f16_bits(w >> 16); }
  static __device__ inline uint32_t pack(float a, float b) { return kBf16 ? pack_bf16(a, b) : pack_f16(a, b); }
  static __device__ inline void from_raw(const R& r, float (&v)[CV]) {
    if constexpr (CV == 1) {
      v[0] = lo(r.h);
    } else {
#pragma unroll
      for (int i = 0; i < CV / 2; ++i) {
        v[2 * i] = lo(r.w[i]);
        v[2 * i + 1] = hi(r.w[i]);
      }
    }
  }
  static __device__ inline void load(const char* p, float (&v)[CV]) {
    from_raw(*reinterpret_cast<const R*>(p), v);
  }
  // acc + sum_i a[i] * b[i]: packed dot products (v_dot2c_f32_bf16 / _f16) on the
  // raw pairs. A product of two 16-bit values is exact in fp32, so this equals
  // widening both and accumulating with FMAs up to fp32 rounding.
  static __device__ inline float dot(const R& a, const R& b, float acc) {
    if constexpr (CV == 1) {
      return fma(lo(a.h), lo(b.h), acc);
    } else {
#pragma unroll
      for (int i = 0; i < CV / 2; ++i) {
        if constexpr (kBf16)
          acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.w[i]),
                                                __builtin_bit_cast(bf16x2_v, b.w[i]), acc, false);
        else
          acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_v, a.w[i]), __builtin_bit_cast(f16x2_v, b.w[i]),
                                       acc, false);
      }
      return acc;
    }
  }
  static __device__ inline void store(char* p, const float (&v)[CV]) {
    R r;
    if constexpr (CV == 1) {
      r.h = static_cast<uint16_t>(pack(v[0], 0.0f));
    } else {
#pragma unroll
      for (int i = 0; i < CV / 2; ++i) r.w[i] = pack(v[2 * i], v[2 * i + 1]);
    }
    *reinterpret_cast<R*>(p) = r;
  }
};
template <int CV> struct Chan<bf16_t, CV> : Chan16<bf16_t, CV> {};
template <int CV> struct Chan<f16_t, CV> : Chan16<f16_t, CV> {};

// ---------------------------------------------------------------------------
// Cross-lane reductions inside the LH lanes of one unit (LH a power of two, the
// unit's lanes contiguous and aligned). Every lane of the wave must call them.

// Units of up to four lanes (bf16 / f16 D = 32 takes four) use DPP quad
// permutations, which stay in the VALU; wider units go through ds_bpermute.
template <int CTRL> __device__ inline float quad_perm(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
constexpr int kQuadXor1 = 0xb1;       // quad_perm [1, 0, 3, 2]
constexpr int kQuadXor2 = 0x4e;       // quad_perm [2, 3, 0, 1]
constexpr int kRowHalfMirror = 0x141;  // lane i of each 8 reads lane 7 - i
constexpr int kRowMirror = 0x140;      // lane i of each 16 reads lane 15 - i

// Sum / max over a unit's lh lanes (a power of two), left in every lane. float units
// of up to 16 lanes use DPP moves: after the quad steps each group of 4 holds its
// total, and a mirror pairs every lane with one of the other group (the sums are
// the same in every lane: each step adds two equal-ordered values).
template <typename A> __device__ inline A unit_sum(A v, int lh) {
  if constexpr (__is_same(A, float)) {
    if (lh <= 4) {
      if (lh >= 2) v += quad_perm<kQuadXor1>(v);
      if (lh >= 4) v += quad_perm<kQuadXor2>(v);
      return v;
    }
    if (lh <= 16) {
      v += quad_perm<kQuadXor1>(v);
      v += quad_perm<kQuadXor2>(v);
      v += quad_perm<kRowHalfMirror>(v);
      if (lh >= 16) v += quad_perm<kRowMirror>(v);
      return v;
    }
  }
  for (int m = 1; m < lh; m <<= 1) v += __shfl_xor(v, m, kWave);
  return v;
}
template <typename A> __device__ inline A unit_max(A v, int lh) {
  if constexpr (__is_same(A, float)) {
    if (lh <= 4) {
      if (lh >= 2) v = fmax(v, quad_perm<kQuadXor1>(v));
      if (lh >= 4) v = fmax(v, quad_perm<kQuadXor2>(v));
      return v;
    }
    if (lh <= 16) {
      v = fmax(v, quad_perm<kQuadXor1>(v));
      v = fmax(v, quad_perm<kQuadXor2>(v));
      v = fmax(v, quad_perm<kRowHalfMirror>(v));
      if (lh >= 16) v = fmax(v, quad_perm<kRowMirror>(v));
      return v;
    }
  }
  for (int m = 1; m < lh; m <<= 1) v = fmax(v, __shfl_xor(v, m, kWave));
  return v;
}

// The sums over a unit's lh lanes (4 or 8) of eight values per lane, reduce-scattered:
// each halving step swaps the half of its values a lane does not keep with its
// partner, so the steps move 4, 2 (and 1) values instead of 8 each. Lane t of the
// unit ends with value t (lh = 8) or values 2 t and 2 t + 1 (lh = 4) in v[0] (v[1]).
template <int CTRL, int N> __device__ inline void halve(float (&v)[8], bool hi) {
#pragma unroll
  for (int j = 0; j < N / 2; ++j) {
    const float send = hi ? v[j] : v[N / 2 + j];
    const float keep = hi ? v[N / 2 + j] : v[j];
    v[j] = keep + quad_perm<CTRL>(send);
  }
}
__device__ inline void unit_reduce_scatter8(float (&v)[8], int lh, int t) {
  if (lh == 8) {
    halve<kRowHalfMirror, 8>(v, (t & 4) != 0);  // lane i pairs with 7 - i
    halve<kQuadXor2, 4>(v, (t & 2) != 0);
    halve<kQuadXor1, 2>(v, (t & 1) != 0);
  } else {
    halve<kQuadXor2, 8>(v, (t & 2) != 0);
    halve<kQuadXor1, 4>(v, (t & 1) != 0);
  }
}

__device__ inline float exp_acc(float x) { return __expf(x); }
__device__ inline double exp_acc(double x) { return exp(x); }

// grad_value[p + i] += w * g[i] for the CV channels at byte address p, with global
// atomics in the value dtype: fp32 and fp64 adds, packed bf16 / f16 pair adds
// (CV >= 2 keeps p 4-byte aligned), and for a single 16-bit channel a 32-bit
// compare-and-swap on the aligned word that holds it (the word never leaves the
// element's page, and the swap leaves the other half as it finds it).
template <typename T, int CV>
__device__ inline void atomic_add_channels(char* p, typename Elem<T>::acc w, const typename Elem<T>::acc (&g)[CV]) {
  if constexpr (std::is_same_v<T, float> || std::is_same_v<T, double>) {
#pragma unroll
    for (int i = 0; i < CV; ++i) unsafeAtomicAdd(reinterpret_cast<T*>(p) + i, w * g[i]);
  } else if constexpr (CV >= 2) {
#pragma unroll
    for (int i = 0; i < CV / 2; ++i) {
      if constexpr (std::is_same_v<T, bf16_t>) {
        const bf16x2_v v = {static_cast<__bf16>(w * g[2 * i]), static_cast<__bf16>(w * g[2 * i + 1])};
        __builtin_amdgcn_global_atomic_fadd_v2bf16(reinterpret_cast<bf16x2_v*>(p) + i, v);
      } else {
        const f16x2_v v = {static_cast<_Float16>(w * g[2 * i]), static_cast<_Float16>(w * g[2 * i + 1])};
        __builtin_amdgcn_global_atomic_fadd_v2f16(reinterpret_cast<f16x2_v*>(p) + i, v);
      }
    }
  } else {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    uint32_t* word = reinterpret_cast<uint32_t*>(a & ~uintptr_t(3));
    const int shift = (a & 2) ? 16 : 0;
    const float add = w * g[0];
    uint32_t old = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (;;) {
      const uint32_t bits = (old >> shift) & 0xffffu;
      float cur;
      uint32_t nb;
      if constexpr (std::is_same_v<T, bf16_t>) {
        cur = __uint_as_float(bits << 16);
        nb = __builtin_bit_cast(uint16_t, static_cast<__bf16>(cur + add));
      } else {
        cur = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
        nb = __builtin_bit_cast(uint16_t, static_cast<_Float16>(cur + add));
      }
      const uint32_t want = (old & ~(0xffffu << shift)) | (nb << shift);
      if (__hip_atomic_compare_exchange_strong(word, &old, want, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT))
        break;
    }
  }
}


// ---------------------------------------------------------------------------
// Problem description, passed by value to every kernel.

struct Problem {
  const char* value;
  const void* shapes;
  const void* starts;
  const char* loc;
  const char* attn;
  char* out;
  const char* grad_out;
  char* grad_value;
  char* grad_loc;
  char* grad_attn;
  int index_i32;
  int B, S, H, D, Q, L, P;
  int lh_log2;          // log2 of lanes per unit
  int units_per_block;  // waves per block * units per wave
  int blocks_per_batch;
  int num_blocks;
  int loc_piece, attn_piece;  // bytes per lane access copying a wave's records to LDS
  int atomic_gv;              // backward: grad_sample scatters grad_value with atomics
  // Backward on the matrix-core owners: levels that share positions of S are sorted
  // too (each level's tiles are its own buckets); the count pass zeroes grad_value
  // (when zero_gv) and the owners add their fp32 sums with atomics.
  int sort_overlap;
  int zero_gv;  // grad_value starts at zero (not accumulated into)
  int es;       // bytes of one value element
  // Softmax backward with grad_sample beside the sort: grad_sample writes every
  // unit's log-sum-exp here (a SoftStat per (b, q, h)) for the grad_value kernel, in
  // place of msda_softmax_stats_kernel. Null otherwise.
  char* stats;
};

// One pyramid level as the kernels use it. A level whose table entry does not fit
// inside the S positions of the value tensor is marked !ok and sampled nowhere, so
// a malformed table cannot make a kernel read or write outside its tensors.
struct alignas(16) Level {
  int h, w, start, ok;
};

// A staged sample: four corner rows (position * H + head inside one batch image,
// below 2^31 since the image holds fewer than 2^31 elements; a row is D elements)
// and four weights (bilinear * attention in the accumulation
// type, fp32 for every 16-bit value dtype; zero for a corner outside the level). In
// the backward the weights slot is reused for the reduced G_c once phase 2 has read
// it.
template <typename A> struct alignas(16) Staged {
  uint32_t off[4];
  A w[4];
};

__device__ inline void load_levels(const Problem& p, Level* levels) {
  for (int i = threadIdx.x; i < p.L; i += blockDim.x) {
    int64_t h, w, st;
    if (p.index_i32) {
      h = static_cast<const int32_t*>(p.shapes)[2 * i];
      w = static_cast<const int32_t*>(p.shapes)[2 * i + 1];
      st = static_cast<const int32_t*>(p.starts)[i];
    } else {
      h = static_cast<const int64_t*>(p.shapes)[2 * i];
      w = static_cast<const int64_t*>(p.shapes)[2 * i + 1];
      st = static_cast<const int64_t*>(p.starts)[i];
    }
    const bool ok = h > 0 && w > 0 && st >= 0 && h <= p.S && w <= p.S && st + h * w <= p.S;
    levels[i] = ok ? Level{int(h), int(w), int(st), 1} : Level{1, 1, 0, 0};
  }
}

// Whether this thread's levels (i = threadIdx.x, + blockDim.x, ...) share positions
// of S with another valid level. The reference's validator calls such a table
// malformed (core/sanitize.py:395-436), but its eager and atomic paths sum every
// level's contribution into a shared element; the backward does the same by
// scattering grad_value with atomics when any level overlaps. Callers OR the
// result over the workgroup with overlap_flag_raise.
__device__ inline bool thread_levels_overlap(const Level* levels, int L) {
  bool any = false;
  for (int i = threadIdx.x; i < L && !any; i += blockDim.x) {
    const Level a = levels[i];
    if (!a.ok) continue;
    const int64_t a0 = a.start, a1 = a0 + int64_t(a.h) * a.w;
    for (int j = 0; j < L; ++j) {
      const Level b = levels[j];
      const int64_t b0 = b.start, b1 = b0 + int64_t(b.h) * b.w;
      if (j != i && b.ok && a0 < b1 && b0 < a1) {
        any = true;
        break;
      }
    }
  }
  return any;
}

// A workgroup's "levels overlap" flag in LDS: cleared by thread 0 before a barrier,
// raised (rarely) by the threads that find an overlap between that barrier and the
// next, read by every thread after the next.
__device__ inline int* overlap_flag() {
  __shared__ int flag;
  return &flag;
}
__device__ inline void overlap_flag_raise(const Level* levels, int L) {
  if (thread_levels_overlap(levels, L)) atomicOr(overlap_flag(), 1);
}

// Geometry of one sample. Contraction is off so that pixel = loc * size - 0.5 and
// the bilinear weights round exactly as the eager reference's separate tensor ops
// do; a fused multiply-add would move samples that sit on a pixel boundary to the
// neighbouring cell and flip their one-sided location gradient.
template <typename A> struct Geom {
  A dx, dy;
  A w00, w01, w10, w11;  // bilinear weights, zero for corners outside the level
  uint32_t off[4];       // corner rows of the image: position * H + head (clamped into the level)
  int ix, iy;            // top-left corner (floor of the pixel coordinates), when in
  bool in;               // the sample counts: -1 <= pixel < size on both axes
  bool m00, m01, m10, m11;
};

template <typename A>
__device__ inline Geom<A> geometry(A lx, A ly, const Level lv, uint32_t head, uint32_t heads) {
#pragma clang fp contract(off)
  Geom<A> g;
  const A W = A(lv.w), H = A(lv.h);
  const A x = lx * W - A(0.5);
  const A y = ly * H - A(0.5);
  const bool in = lv.ok && x >= A(-1) && x < W && y >= A(-1) && y < H;
  const A xf = in ? floor(x) : A(0);
  const A yf = in ? floor(y) : A(0);
  g.dx = in ? x - xf : A(0);
  g.dy = in ? y - yf : A(0);
  const int ix = int(xf), iy = int(yf);
  g.ix = ix;
  g.iy = iy;
  g.in = in;
  const bool mx0 = in && ix >= 0, mx1 = in && ix + 1 < lv.w;
  const bool my0 = in && iy >= 0, my1 = in && iy + 1 < lv.h;
  g.m00 = mx0 && my0;
  g.m01 = mx1 && my0;
  g.m10 = mx0 && my1;
  g.m11 = mx1 && my1;
  const int cx0 = max(ix, 0), cx1 = min(ix + 1, lv.w - 1);
  const int cy0 = max(iy, 0), cy1 = min(iy + 1, lv.h - 1);
  const uint32_t base = uint32_t(lv.start) * heads + head;
  const uint32_t r0 = uint32_t(cy0 * lv.w), r1 = uint32_t(cy1 * lv.w);
  g.off[0] = base + (r0 + uint32_t(cx0)) * heads;
  g.off[1] = base + (r0 + uint32_t(cx1)) * heads;
  g.off[2] = base + (r1 + uint32_t(cx0)) * heads;
  g.off[3] = base + (r1 + uint32_t(cx1)) * heads;
  const A one(1);
  g.w00 = g.m00 ? (one - g.dx) * (one - g.dy) : A(0);
  g.w01 = g.m01 ? g.dx * (one - g.dy) : A(0);
  g.w10 = g.m10 ? (one - g.dx) * g.dy : A(0);
  g.w11 = g.m11 ? g.dx * g.dy : A(0);
  return g;
}

// XCD-aware renumbering: hardware workgroup i runs on XCD i % 8. Returns a logical
// index such that each XCD runs one contiguous range of logical workgroups, so
// workgroups that share cache lines (neighbouring queries, the heads of one query)
// share that XCD's L2.
__device__ inline int xcd_logical_block() {
  const int n = int(gridDim.x), per = n / kXcds, rem = n % kXcds;
  const int xcd = int(blockIdx.x) % kXcds, slot = int(blockIdx.x) / kXcds;
  return xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

// Grid of (group, head) workgroups where the heads of a group should share an L2:
// group g runs on XCD g % 8, its H heads back to back; groups reach each XCD in
// increasing order. The grid is padded to a multiple of 8 * H; returns false for
// the padding.
__device__ inline bool xcd_group_block(int H, int ngroups, int* group, int* head) {
  const int xcd = int(blockIdx.x) % kXcds, k = int(blockIdx.x) / kXcds;
  *head = k % H;
  *group = (k / H) * kXcds + xcd;
  return *group < ngroups;
}

int64_t xcd_group_grid(int64_t H, int64_t ngroups) {
  return (ngroups + kXcds - 1) / kXcds * kXcds * H;
}

// Block-invariant facts of one lane.
struct LaneMap {
  int lane, wave, t, uw, lh, uw_count;
  int b, unit;       // batch index and q * H + h inside the batch
  bool unit_ok;      // unit < Q * H
  int h;
  int64_t gunit;     // (b * Q + q) * H + h
};

__device__ inline LaneMap map_lane(const Problem& p) {
  LaneMap m;
  m.lane = threadIdx.x & (kWave - 1);
  m.wave = threadIdx.x / kWave;
  m.lh = 1 << p.lh_log2;
  m.uw_count = kWave >> p.lh_log2;
  m.t = m.lane & (m.lh - 1);
  m.uw = m.lane >> p.lh_log2;
  const int blk = xcd_logical_block();
  m.b = blk / p.blocks_per_batch;
  m.unit = (blk - m.b * p.blocks_per_batch) * p.units_per_block + m.wave * m.uw_count + m.uw;
  m.unit_ok = m.unit < p.Q * p.H;
  m.h = m.unit_ok ? m.unit % p.H : 0;
  m.gunit = int64_t(m.b) * p.Q * p.H + m.unit;
  return m;
}

// Keeps the compiler from moving this wave's LDS accesses across it. The LDS
// executes one wave's instructions in order, so lanes of a wave then see each
// other's earlier writes without a barrier.
__device__ inline void wave_lds_order() { __asm__ volatile("" ::: "memory"); }

// Copies bytes from global memory to LDS, `piece` bytes (16, 8, 4, 2 or 1, dividing
// `bytes` and the alignment of both ends) per lane and step.
__device__ inline void copy_pieces(unsigned char* dst, const char* src, int bytes, int piece, int lane) {
  if (piece == 16) {
    for (int i = lane * 16; i < bytes; i += kWave * 16)
      *reinterpret_cast<u32x4_v*>(dst + i) = *reinterpret_cast<const u32x4_v*>(src + i);
  } else if (piece == 8) {
    for (int i = lane * 8; i < bytes; i += kWave * 8)
      *reinterpret_cast<u32x2_v*>(dst + i) = *reinterpret_cast<const u32x2_v*>(src + i);
  } else if (piece == 4) {
    for (int i = lane * 4; i < bytes; i += kWave * 4)
      *reinterpret_cast<uint32_t*>(dst + i) = *reinterpret_cast<const uint32_t*>(src + i);
  } else if (piece == 2) {
    for (int i = lane * 2; i < bytes; i += kWave * 2)
      *reinterpret_cast<uint16_t*>(dst + i) = *reinterpret_cast<const uint16_t*>(src + i);
  } else {
    for (int i = lane; i < bytes; i += kWave) dst[i] = static_cast<unsigned char>(src[i]);
  }
}

// Bytes of one wave's LDS copy of its units' locations and weights (each part a
// multiple of 16).
__device__ __host__ inline int unit_raw_bytes(int uw_count, int LP, int loc_es, int es) {
  return ((uw_count * LP * 2 * loc_es + 15) & ~15) + ((uw_count * LP * es + 15) & ~15);
}

// A lane's unit's locations and weights in the wave's LDS copy.
struct UnitRaw {
  const unsigned char* loc;
  const unsigned char* attn;
};

// The wave's units are consecutive (b, q, h), so their locations and their weights
// are two contiguous ranges: the wave copies both to its part of `raw_base` (which
// follows the staged records of every wave) with wide coalesced loads, instead of
// one 2- to 8-byte load per sample and coordinate. The copy is complete for the
// other lanes after the next workgroup barrier.
template <typename T, typename TL>
__device__ inline UnitRaw copy_unit_records(const Problem& p, const LaneMap& m, unsigned char* raw_base) {
  constexpr int ES = Elem<T>::size;
  const int LP = p.L * p.P;
  const int loc_unit = LP * 2 * int(sizeof(TL)), attn_unit = LP * ES;
  const int loc_wave = (m.uw_count * loc_unit + 15) & ~15;
  unsigned char* lds_loc = raw_base + size_t(m.wave) * size_t(unit_raw_bytes(m.uw_count, LP, int(sizeof(TL)), ES));
  unsigned char* lds_attn = lds_loc + loc_wave;
  const int first = m.unit - m.uw;  // the wave's first unit in its batch image
  const int n = max(0, min(m.uw_count, p.Q * p.H - first));
  const int64_t g0 = int64_t(m.b) * p.Q * p.H + first;
  copy_pieces(lds_loc, p.loc + g0 * loc_unit, n * loc_unit, p.loc_piece, m.lane);
  copy_pieces(lds_attn, p.attn + g0 * attn_unit, n * attn_unit, p.attn_piece, m.lane);
  return UnitRaw{lds_loc + m.uw * loc_unit, lds_attn + m.uw * attn_unit};
}

// The address of a lane's channels in row `row` (position * H + head) of an image:
// 64-bit, so an image may hold up to 2^31 elements (2^33 bytes for float).
__device__ inline const char* row_at(const char* img, uint32_t row, uint32_t row_bytes, uint32_t lane_bytes) {
  return img + (uint64_t(row) * row_bytes + lane_bytes);
}
__device__ inline char* row_at(char* img, uint32_t row, uint32_t row_bytes, uint32_t lane_bytes) {
  return img + (uint64_t(row) * row_bytes + lane_bytes);
}

// Phase 1, shared by both directions: stage every sample of the lane's unit and
// return the unit's softmax statistics (max and 1 / sum of exp), if any.
template <typename T, typename TL, bool SOFTMAX>
__device__ inline void stage_samples(const Problem& p, const LaneMap& m, const Level* levels,
                                     const UnitRaw& raw, Staged<typename Elem<T>::acc>* wst,
                                     typename Elem<T>::acc& smax,
                                     typename Elem<T>::acc& sinv,
                                     typename Elem<T>::acc* ssum = nullptr) {
  using A = typename Elem<T>::acc;
  constexpr int ES = Elem<T>::size;
  const int LP = p.L * p.P;
  const TL* loc = reinterpret_cast<const TL*>(raw.loc);
  const T* attn = reinterpret_cast<const T*>(raw.attn);
  smax = A(0);
  sinv = A(1);
  if constexpr (SOFTMAX) {
    A mx = -INFINITY;
    if (m.unit_ok)
      for (int s = m.t; s < LP; s += m.lh) mx = fmax(mx, load_acc(attn + s));
    mx = unit_max(mx, m.lh);
    A sum(0);
    if (m.unit_ok)
      for (int s = m.t; s < LP; s += m.lh) sum += exp_acc(load_acc(attn + s) - mx);
    sum = unit_sum(sum, m.lh);
    smax = mx;
    sinv = A(1) / sum;
    if (ssum) *ssum = sum;
  }
  if (!m.unit_ok) return;
  for (int s = m.t; s < LP; s += m.lh) {
    const Geom<A> g = geometry<A>(load_acc(loc + 2 * s), load_acc(loc + 2 * s + 1),
                                  levels[s / p.P], uint32_t(m.h), uint32_t(p.H));
    A a = load_acc(attn + s);
    if constexpr (SOFTMAX) a = exp_acc(a - smax) * sinv;
    Staged<A> st;
#pragma unroll
    for (int c = 0; c < 4; ++c) st.off[c] = g.off[c];
    // A corner outside the level weighs exactly zero, whatever the attention weight
    // (0 * inf would be NaN): the reference skips such corners.
    st.w[0] = g.m00 ? g.w00 * a : A(0);
    st.w[1] = g.m01 ? g.w01 * a : A(0);
    st.w[2] = g.m10 ? g.w10 * a : A(0);
    st.w[3] = g.m11 ? g.w11 * a : A(0);
    wst[s * m.uw_count + m.uw] = st;
  }
}

// ---------------------------------------------------------------------------
// Forward.

template <typename T, typename TL, int CV, bool SOFTMAX>
__global__ __launch_bounds__(kWave * kMaxWavesPerBlock) void msda_forward_kernel(const Problem p) {
  using A = typename Elem<T>::acc;
  constexpr int ES = Elem<T>::size;
  extern __shared__ __align__(16) unsigned char smem[];
  Level* levels = reinterpret_cast<Level*>(smem);
  const LaneMap m = map_lane(p);
  const int LP = p.L * p.P;
  constexpr size_t kRec = sizeof(Staged<A>);
  Staged<A>* wst = reinterpret_cast<Staged<A>*>(smem + sizeof(Level) * p.L + kRec * m.wave * m.uw_count * LP);
  const size_t raw_at = (sizeof(Level) * p.L + kRec * (blockDim.x / kWave) * m.uw_count * LP + 15) & ~size_t(15);
  const UnitRaw raw = copy_unit_records<T, TL>(p, m, smem + raw_at);
  load_levels(p, levels);
  __syncthreads();
  A smax, sinv;
  stage_samples<T, TL, SOFTMAX>(p, m, levels, raw, wst, smax, sinv);
  __syncthreads();

  if (!m.unit_ok || m.t * CV >= p.D) return;
  const char* img = p.value + int64_t(m.b) * p.S * p.H * p.D * ES;
  const uint32_t row_bytes = uint32_t(p.D * ES), lane_bytes = uint32_t(m.t * CV * ES);
  A acc[CV];
#pragma unroll
  for (int i = 0; i < CV; ++i) acc[i] = A(0);
  // Every corner value is widened to the accumulation type and multiplied by its
  // weight (attention * bilinear, kept in that type) into the sum, as the
  // reference's kernels do with their fp32 accumulator.
#pragma unroll 2
  for (int s = 0; s < LP; ++s) {
    const Staged<A> st = wst[s * m.uw_count + m.uw];
    A v[4][CV];
#pragma unroll
    for (int c = 0; c < 4; ++c) Chan<T, CV>::load(row_at(img, st.off[c], row_bytes, lane_bytes), v[c]);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int i = 0; i < CV; ++i) acc[i] = fma(st.w[c], v[c][i], acc[i]);
  }
  Chan<T, CV>::store(p.out + (m.gunit * p.D + m.t * CV) * ES, acc);
}

// ---------------------------------------------------------------------------
// Backward.
//
// grad_value is computed owner-side: every element has exactly one writer, which
// sums its contributions in fp32 (fp64 for double) registers and stores once, so
// there are no atomics on grad_value, no zero-fill and no float32 copy. The
// location and weight gradients are sample-parallel like the forward. Kernels, in
// stream order:
//
//   msda_bucket_kernel<COUNT>  Counting sort of the samples of every (b, h) by the
//   msda_bucket_scan_kernel    level tile that holds their top-left corner (tiles
//   msda_bucket_kernel<PLACE>  are described below). Per workgroup the counts are
//                              aggregated with LDS integer atomics and published with
//                              one global atomic per touched bucket; the scan turns
//                              counts into offsets; the place pass writes every
//                              in-range sample's index into its bucket. The bucket
//                              offsets live in grad_attention_weights and the sample
//                              indices in grad_sampling_locations, both overwritten
//                              later by msda_grad_sample_kernel, so the backward
//                              needs no memory beyond its outputs.
//   msda_softmax_stats_kernel  Softmax only: every (b, q, h)'s log-sum-exp.
//   msda_grad_value_mfma_kernel  The owners on the matrix cores (described below,
//                              with the choice between the two owner kernels); also
//                              zeroes grad_value at positions no valid level covers.
//   msda_gap_zero_kernel       That zeroing, for the VALU owner kernel.
//   msda_grad_value_kernel     The VALU owners (float64, other D, and the fallback):
//                              one tile per workgroup (loop): reads the buckets that
//                              can reach the tile, stages their grad_out rows in
//                              LDS, sorts their corner records by position (LDS
//                              integer counting sort) and accumulates
//                              weight * grad_out into registers owned per
//                              (position, channel group). Then one plain store per
//                              element.
//   msda_grad_sample_kernel    Location and weight gradients, sample-parallel.
//
// Tiles. Level l is cut into rectangles of th x tw positions (at most `cap`, the
// positions one workgroup holds in registers). The target area follows the level's
// expected fan-in (4 Q P corner records spread over h * w positions) so that tiles
// carry similar numbers of records; it is never below `amin`, so a level has at most
// 3 h w / amin + 1 tiles. A sample is filed under the tile of its top-left corner
// (clamped to 0) with a sub-bucket that says whether its corners reach into the
// right-hand tile (1), the tile below (3), both (2) or neither (0). The owner of a
// tile reads its own four sub-buckets, sub-buckets 1-2 of its left neighbour, 2-3 of
// the tile above and 2 of the tile above-left: exactly the samples with a corner in
// the tile.
//
// When the scratch cannot hold the bucket offsets (few samples and many tiles) the
// bucketing is skipped and every tile owner scans all Q * P samples of its level
// instead; both paths give the same result.

constexpr int kOwnerThreads = 256;
constexpr int kOwnerItems = 4;      // (position, channel group) items per thread
constexpr int kOwnerChunks = 4;     // grad_out pieces one thread stages per batch
constexpr int kBucketThreads = 256;
constexpr int kBucketSamples = 32;  // samples per thread in the bucketing kernels
constexpr int kBucketSamplesSmall = 4;  // the same for small calls (a short latency chain per thread)
constexpr int kBucketBatch = 8;     // of which loaded together (at most)
constexpr int kTargetRecords = 8192;
// A level takes 4 x 4 tiles below this many 8 x 8 tasks (B H tiles; about 1.5 per CU:
// more overlap with other levels' work, as at config 4's 512) and from this many
// K-blocks per 8 x 8 task.
constexpr int kSmallTileTasks = 384;
constexpr int kSmallTileKBlocks = 24;
constexpr int kBucketLdsKeys = 8192;  // LDS bucket counters of the bucketing kernels (32 KB)
// Samples per (b, h) up to which the sort runs in one launch (msda_bucket_small_kernel).
constexpr int64_t kSmallSortSamples = int64_t(1) << 14;
constexpr int kMaxOrderedLevels = 64;
// Scratch ints after the bucket rows for the matrix-core kernel's kXcds work-queue
// counters, each on its own 128-byte line (plus the slack to align the first).
constexpr int kQueueLine = 32;
constexpr int kQueueInts = (kXcds + 1) * kQueueLine;

// Unsigned 32-bit division by a divisor fixed per launch: one multiply-high, an
// add and two shifts (Granlund and Montgomery, "Division by invariant integers
// using multiplication", 1994, section 4) instead of the ~30-instruction software
// division. Exact for every dividend below 2^32.
struct FastDiv {
  uint32_t d, m;
  int s;
};

FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{d, 0u, 0};
  if (d <= 1) return f;
  int l = 0;
  while ((uint64_t(1) << l) < d) ++l;  // ceil(log2 d)
  f.m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
  f.s = l - 1;
  return f;
}

__device__ inline uint32_t fdiv(uint32_t n, const FastDiv& f) {
  if (f.d <= 1) return n;
  const uint32_t t = __umulhi(f.m, n);
  return (t + ((n - t) >> 1)) >> f.s;
}

struct BwdGeom {
  int cap;          // positions per tile at most (power of two)
  int amin;         // smallest tile area (power of two)
  int groups;       // G = D / CVR channel groups per position
  int nb;           // samples per owner batch (power of two, <= kOwnerThreads)
  int nw;           // owner workgroups per (b, h)
  int keys_lds;     // bucket counters the bucketing kernels' LDS holds
  int64_t keys_alloc;  // bucket counters per (b, h) the scratch holds; 0: no bucketing
  int64_t region;   // entries per (b, h): Q * L * P
  FastDiv div_lp;   // by L * P
  FastDiv div_p;    // by P
  int sub_log2;     // > 0: tiles are 2^sub_log2 square (the matrix-core grad_value)
  int small_tiles;  // matrix-core grad_value: levels with few heavy tiles take 4 x 4 tiles
  int group4;       // samples go in groups of 4 of one query and level (L P and P multiples of 4)
  FastDiv div_gpq;  // by L * P / 4, groups per query
  FastDiv div_gpl;  // by P / 4, groups per level
  int key_bytes;    // 2 or 4: the count pass saves every sample's key in the grad_value
                    // scratch for the place pass; 0: the place pass recomputes them
  int chunks;       // > 0: the grouped passes may keep per-workgroup counts (chunk_counts,
                    // `chunks` workgroups per (b, h)) for the scan to turn into
                    // per-workgroup bucket offsets, with no global atomics and no clear;
                    // every kernel decides the same way with chunked_sort()
};

struct LevelTiles {
  int lh, lw;     // log2 of the tile height and width
  int ntx, nty;   // tiles across and down
  int base;       // first tile of the level
};

__device__ __host__ inline int pow2_floor(int64_t v) {
  int r = 1;
  while (int64_t(r) * 2 <= v && r < (1 << 30)) r *= 2;
  return r;
}

__device__ inline int log2_ceil(int v) {
  int r = 0;
  while ((1 << r) < v && r < 30) ++r;
  return r;
}

// Tiles of every level (one thread). Tile sides are powers of two, so that tiles
// and sub-buckets follow from shifts and masks; a tile may reach past the level's
// right or bottom edge. Returns the tile count of one (b, h), or -1 when it exceeds
// 2^29.
__device__ inline int64_t plan_tiles(const Problem& p, const BwdGeom& bg, const Level* levels,
                                     LevelTiles* lt) {
  int64_t total = 0;
  const int64_t records = 4 * int64_t(p.Q) * p.P;
  for (int l = 0; l < p.L; ++l) {
    const Level lv = levels[l];
    LevelTiles t{0, 0, 0, 0, int(total)};
    if (lv.ok && bg.sub_log2 > 0) {
      int side = bg.sub_log2;
      // A level with few tasks of many candidates (a coarse level of a small call)
      // takes 4 x 4 tiles, one MFMA sub-tile each: four times the tasks, each with
      // about a third of the candidates, so that they do not run long after the other
      // levels' tasks (the call waits for its longest task).
      if (bg.small_tiles) {
        const int64_t t8 = int64_t((lv.w + 7) >> 3) * ((lv.h + 7) >> 3);
        const int64_t kblocks = int64_t(p.Q) * p.P * 13 / (10 * 64 * t8);  // per 8 x 8 task, expected
        if (int64_t(p.B) * p.H * t8 < kSmallTileTasks && kblocks >= kSmallTileKBlocks) side = 2;
      }
      t.lw = t.lh = side;
      t.ntx = (lv.w + (1 << t.lw) - 1) >> t.lw;
      t.nty = (lv.h + (1 << t.lh) - 1) >> t.lh;
    } else if (lv.ok) {
      const int64_t hw = int64_t(lv.h) * lv.w;
      const int64_t want = records > 0 ? int64_t(kTargetRecords) * hw / records : bg.cap;
      const int a = pow2_floor(std::min<int64_t>(std::max<int64_t>(want, bg.amin), bg.cap));
      int tw0 = 1;
      while (tw0 * tw0 < a) tw0 *= 2;
      const int wcap = 1 << log2_ceil(lv.w), hcap = 1 << log2_ceil(lv.h);
      int tw = min(wcap, tw0);
      const int th = min(hcap, max(1, a / tw));
      tw = min(wcap, max(tw, a / th));
      t.lw = log2_ceil(tw);
      t.lh = log2_ceil(th);
      t.ntx = (lv.w + tw - 1) >> t.lw;
      t.nty = (lv.h + th - 1) >> t.lh;
    }
    lt[l] = t;
    total += int64_t(t.ntx) * t.nty;
    if (total > (int64_t(1) << 29)) return -1;
  }
  return total;
}

// The bucket key of an in-range sample at level l: 4 * tile + sub-bucket.
__device__ inline int bucket_key(const LevelTiles& t, int ix, int iy, const Level& lv) {
  const int cx = max(ix, 0), cy = max(iy, 0);
  const int tile = t.base + (cy >> t.lh) * t.ntx + (cx >> t.lw);
  const bool sx = ix >= 0 && ix + 1 < lv.w && ((ix + 1) & ((1 << t.lw) - 1)) == 0;
  const bool sy = iy >= 0 && iy + 1 < lv.h && ((iy + 1) & ((1 << t.lh) - 1)) == 0;
  const int sub = sx ? (sy ? 2 : 1) : (sy ? 3 : 0);
  return 4 * tile + sub;
}

// Workgroup barrier for LDS traffic only: the fences are restricted to the local
// address space, so global loads issued before it stay in flight across it.
__device__ inline void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Inclusive prefix sum of v over the wave with DPP lane moves (VALU, no LDS round
// trips): shifts by 1, 2, 4, 8 inside each row of 16 lanes, then row broadcasts of
// lane 15 and lane 31 carry the row totals forward.
__device__ inline int wave_inclusive_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

// Exclusive prefix sum of one value per thread over the workgroup; *total gets the
// sum. `wave_sums` holds one int per wave. Contains two barriers.
__device__ inline int block_exclusive_scan(int v, int* wave_sums, int* total) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int nwaves = int(blockDim.x) / kWave;
  const int inc = wave_inclusive_scan(v);
  if (lane == kWave - 1) wave_sums[wave] = inc;
  lds_barrier();
  int before = 0, all = 0;
  for (int w = 0; w < nwaves; ++w) {
    const int ws = wave_sums[w];
    before += w < wave ? ws : 0;
    all += ws;
  }
  lds_barrier();
  *total = all;
  return before + inc - v;
}

// The normalized weight of sample s of a unit: the raw weight, or its softmax over
// the unit's L * P logits (max first, so -inf logits are safe).
template <typename T, bool SOFTMAX>
__device__ inline typename Elem<T>::acc unit_weight(const T* unit_attn, int LP, int s) {
  using A = typename Elem<T>::acc;
  if constexpr (!SOFTMAX) {
    return load_acc(unit_attn + s);
  } else {
    A mx = -INFINITY;
    for (int i = 0; i < LP; ++i) mx = fmax(mx, load_acc(unit_attn + i));
    A sum(0);
    for (int i = 0; i < LP; ++i) sum += exp_acc(load_acc(unit_attn + i) - mx);
    return exp_acc(load_acc(unit_attn + s) - mx) / sum;
  }
}

// Shared set-up of the bucketing kernels and the owners: the level table and the
// tiles in LDS. Returns the tile count of one (b, h), or -1 when there are too many
// tiles. When valid levels overlap (`overlap` then says so), the matrix-core owners
// take them too (sort_overlap) and add into a zeroed grad_value; otherwise -1: the
// sort and the owners stand aside, and msda_grad_sample_kernel scatters grad_value
// with atomics.
__device__ inline int64_t load_tiles(const Problem& p, const BwdGeom& bg, Level* levels,
                                     LevelTiles* lt, int64_t* total_out, bool* overlap = nullptr) {
  if (threadIdx.x == 0) *overlap_flag() = 0;
  load_levels(p, levels);
  __syncthreads();
  overlap_flag_raise(levels, p.L);
  if (threadIdx.x == 0) *total_out = plan_tiles(p, bg, levels, lt);
  __syncthreads();
  const bool any = *overlap_flag() != 0;
  if (overlap) *overlap = any;
  return any && !p.sort_overlap ? -1 : *total_out;
}

// The per-workgroup count rows of the chunked bucket sort, nkeys ints for each
// (b, h, workgroup), after the bucket rows and the matrix-core kernel's queue
// counters; then the bucket totals, nkeys ints per (b, h).
__device__ inline int* chunk_counts(int* buckets, const Problem& p, int64_t nkeys) {
  return buckets + ((int64_t(p.B) * p.H * nkeys + 31) & ~int64_t(31)) + kQueueInts;
}
__device__ inline int* chunk_totals(int* buckets, const Problem& p, const BwdGeom& bg, int64_t nkeys) {
  return chunk_counts(buckets, p, nkeys) + int64_t(p.B) * p.H * bg.chunks * nkeys;
}

// Whether the bucket sort keeps per-workgroup counts, from the device's tile count:
// every bucket fits the bucketing kernels' LDS counters, and the scratch holds the
// bucket rows, the queue counters and the count rows.
__device__ inline bool chunked_sort(const Problem& p, const BwdGeom& bg, int64_t nkeys) {
  if (bg.chunks <= 0 || nkeys > bg.keys_lds) return false;
  const int64_t bh = int64_t(p.B) * p.H;
  const int64_t need = ((bh * nkeys + 31) & ~int64_t(31)) + kQueueInts + bh * (bg.chunks + 1) * nkeys;
  return need <= bh * bg.keys_alloc;
}

// Whether the bucket counters of every (b, h) and, after them, the matrix-core
// kernel's work-queue counters fit the scratch. The host picks the matrix-core
// kernel from an estimate of the tile count; the kernels that touch the queue
// counters check the real count here, and the VALU owner kernel runs instead when
// they do not fit.
__device__ inline bool queue_fits(const Problem& p, const BwdGeom& bg, int64_t nkeys) {
  const int64_t bh = int64_t(p.B) * p.H;
  return nkeys <= bg.keys_alloc && bh * nkeys + kQueueInts <= bh * bg.keys_alloc;
}

// Per-unit softmax statistics for the grad_value kernels: lse = max + log(sum of
// exp(logit - max)) of every (b, q, h), written by msda_softmax_stats_kernel after
// the place pass (over the per-workgroup counts, done with by then), where the
// scratch has room. A candidate's weight is then exp(logit - lse): one logit and one
// 4-byte statistics load instead of a pass over the unit's L * P logits.
template <typename A> struct SoftStat {
  A lse;
};
template <typename A>
__device__ inline SoftStat<A>* softmax_stats(int* buckets, const Problem& p, int64_t nkeys) {
  return reinterpret_cast<SoftStat<A>*>(chunk_counts(buckets, p, nkeys));
}
template <typename A>
__device__ inline bool softmax_stats_fit(const Problem& p, const BwdGeom& bg, int64_t nkeys, const int* buckets) {
  const int64_t bh = int64_t(p.B) * p.H;
  const int64_t ints = int64_t(sizeof(SoftStat<A>) / sizeof(int)) * bh * p.Q;
  const int64_t need = ((bh * nkeys + 31) & ~int64_t(31)) + kQueueInts + ints;
  const uintptr_t at = reinterpret_cast<uintptr_t>(softmax_stats<A>(const_cast<int*>(buckets), p, nkeys));
  return need <= bh * bg.keys_alloc && at % alignof(SoftStat<A>) == 0;
}

// The gradients of one sample from its corner dots G_c = <grad_out, value at corner
// c> (ignored for corners outside the level): with respect to its weight,
// sum_c bilinear_c G_c; with respect to its normalized location, the attention
// weight a times the derivatives of the bilinear weights (pixel units, scaled by the
// level's width and height). A sample outside the level has no corner: its location
// gradient is zero whatever its weight (the reference skips it). Without
// contraction, as the eager reference's separate tensor operations round.
template <typename A>
__device__ inline void sample_grads(const Geom<A>& ge, A a, const Level& lv, A g00, A g01, A g10, A g11, A* gx,
                                    A* gy, A* gpv) {
#pragma clang fp contract(off)
  const A G00 = ge.m00 ? g00 : A(0);
  const A G01 = ge.m01 ? g01 : A(0);
  const A G10 = ge.m10 ? g10 : A(0);
  const A G11 = ge.m11 ? g11 : A(0);
  const A one(1);
  *gpv = ge.w00 * G00 + ge.w01 * G01 + ge.w10 * G10 + ge.w11 * G11;
  *gx = ge.in ? a * A(lv.w) * ((one - ge.dy) * (G01 - G00) + ge.dy * (G11 - G10)) : A(0);
  *gy = ge.in ? a * A(lv.h) * ((one - ge.dx) * (G10 - G00) + ge.dx * (G11 - G01)) : A(0);
}

// Overlapping levels on the matrix-core owners: the count pass zeroes grad_value
// (its workgroups, grid-stride, 16 bytes a thread) before the owners add into it; the
// keys then stay out of grad_value and the place pass recomputes them.
__device__ inline void zero_grad_value(const Problem& p) {
  const int64_t bytes = int64_t(p.B) * p.S * p.H * p.D * p.es;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  const int64_t first = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (bytes % 16 == 0 && reinterpret_cast<uintptr_t>(p.grad_value) % 16 == 0) {
    const u32x4_v zero = {0u, 0u, 0u, 0u};
    for (int64_t i = first; i < bytes / 16; i += stride) reinterpret_cast<u32x4_v*>(p.grad_value)[i] = zero;
  } else {
    for (int64_t i = first; i < bytes / 2; i += stride) reinterpret_cast<uint16_t*>(p.grad_value)[i] = 0;
  }
}

// Counting (PLACE = false) or placing (PLACE = true) pass of the bucket sort.
// Workgroup: kBucketThreads * SPT consecutive samples (q, l, p) of one
// (b, h). `buckets` holds one counter per bucket and (b, h): counts after the count
// pass, exclusive offsets after the scan, and bucket ends after the place pass.
// The workgroup first counts its samples per bucket in LDS and publishes each
// non-empty count with one global atomic; the place pass gets its range of every
// bucket back from that atomic and hands out slots from it with LDS atomics while
// it recomputes the keys.
template <typename TL, bool PLACE, int SPT>
__global__ __launch_bounds__(kBucketThreads) void msda_bucket_kernel(const Problem p, const BwdGeom bg,
                                                                     int* __restrict__ buckets,
                                                                     uint32_t* __restrict__ entries,
                                                                     int chunks_per_bh) {
  using A = typename Elem<TL>::acc;  // the precision the owner kernel's geometry uses
  extern __shared__ __align__(16) unsigned char smem[];
  Level* levels = reinterpret_cast<Level*>(smem);
  LevelTiles* lt = reinterpret_cast<LevelTiles*>(smem + sizeof(Level) * size_t(p.L));
  const size_t head = ((sizeof(Level) + sizeof(LevelTiles)) * size_t(p.L) + 15) & ~size_t(15);
  int64_t* total = reinterpret_cast<int64_t*>(smem + head);
  int* hist = reinterpret_cast<int*>(smem + head + 16);
  bool overlap = false;
  const int64_t ntiles = load_tiles(p, bg, levels, lt, total, &overlap);
  const int64_t nkeys = 4 * ntiles;
  if (ntiles < 0 || nkeys > bg.keys_alloc) return;  // no bucketing: the owners scan
  if (!PLACE && overlap && p.zero_gv) zero_grad_value(p);
  const bool in_lds = nkeys <= bg.keys_lds;
  // Groups (b, chunk), the heads of a group on one XCD: they share the cache lines of
  // their queries' locations.
  int group, h;
  if (!xcd_group_block(p.H, p.B * chunks_per_bh, &group, &h)) return;
  const int chunk = group % chunks_per_bh;
  const int b = group / chunks_per_bh;
  const int bh = b * p.H + h;
  const int LP = p.L * p.P;
  const int64_t nsamples = int64_t(p.Q) * LP;
  int* bucket_row = buckets + int64_t(bh) * nkeys;
  uint32_t* out = entries + int64_t(bh) * bg.region;
  const TL* loc_all = reinterpret_cast<const TL*>(p.loc);
  const int64_t j0 = int64_t(chunk) * kBucketThreads * SPT;
  constexpr int kBatch = SPT < kBucketBatch ? SPT : kBucketBatch;

  // Bucket of sample j of (b, h), or -1 when it is out of range (or j past the end).
  auto key_of = [&](int64_t j) __attribute__((always_inline)) -> int {
    if (j >= nsamples) return -1;
    const uint32_t j32 = uint32_t(j);  // Q * L * P < 2^32
    const int q = int(fdiv(j32, bg.div_lp)), s = int(j32 - uint32_t(q) * uint32_t(LP));
    const int l = int(fdiv(uint32_t(s), bg.div_p));
    const Level lv = levels[l];
    const TL* lc = loc_all + (((int64_t(b) * p.Q + q) * p.H + h) * LP + s) * 2;
    const Geom<A> g = geometry<A>(load_acc(lc), load_acc(lc + 1), lv, 0u, 1u);
    return g.in ? bucket_key(lt[l], g.ix, g.iy, lv) : -1;
  };

  if (!in_lds) {
    // Too many buckets for LDS: one global atomic per sample.
    for (int k = 0; k < SPT; k += kBatch) {
      int key[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) key[i] = key_of(j0 + (k + i) * kBucketThreads + threadIdx.x);
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        if (key[i] < 0) continue;
        const int at = atomicAdd(&bucket_row[key[i]], 1);
        if constexpr (PLACE) out[at] = uint32_t(j0 + (k + i) * kBucketThreads + threadIdx.x);
      }
    }
    return;
  }
  for (int k = threadIdx.x; k < nkeys; k += kBucketThreads) hist[k] = 0;
  __syncthreads();
  for (int k = 0; k < SPT; k += kBatch) {
    int key[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) key[i] = key_of(j0 + (k + i) * kBucketThreads + threadIdx.x);
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      if (key[i] >= 0) atomicAdd(&hist[key[i]], 1);
  }
  __syncthreads();
  for (int k = threadIdx.x; k < nkeys; k += kBucketThreads) {
    const int c = hist[k];
    if (c > 0) {
      const int at = atomicAdd(&bucket_row[k], c);
      if constexpr (PLACE) hist[k] = at;  // becomes this workgroup's cursor in bucket k
    }
  }
  if constexpr (PLACE) {
    __syncthreads();
    for (int k = 0; k < SPT; k += kBatch) {
      int key[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) key[i] = key_of(j0 + (k + i) * kBucketThreads + threadIdx.x);
#pragma unroll
      for (int i = 0; i < kBatch; ++i)
        if (key[i] >= 0) out[atomicAdd(&hist[key[i]], 1)] = uint32_t(j0 + (k + i) * kBucketThreads + threadIdx.x);
    }
  }
}

// The bucket key of a sample at level lv (-1: out of range), with the same pixel
// map as the kernels that own the tiles.
template <typename A>
__device__ inline int sample_key(A lx, A ly, const Level& lv, const LevelTiles& t) {
#pragma clang fp contract(off)
  const A x = lx * A(lv.w) - A(0.5);
  const A y = ly * A(lv.h) - A(0.5);
  const bool in = lv.ok && x >= A(-1) && x < A(lv.w) && y >= A(-1) && y < A(lv.h);
  return in ? bucket_key(t, int(floor(x)), int(floor(y)), lv) : -1;
}

// Slots for the four samples of a group (points p .. p + 3 of one query and level)
// from the bucket cursors `cur`: samples that share a bucket get consecutive slots
// from one atomic, so a tile's candidate list holds a query's points of one level
// side by side, and the grad_value kernel's lanes then read the same grad_out row
// and location line together. Keys < 0 get no slot.
template <typename Cursor>
__device__ inline void group_slots(const int (&key)[4], Cursor* cur, int (&slot)[4]) {
#pragma unroll
  for (int c = 0; c < 4; ++c) slot[c] = -1;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    bool first = key[c] >= 0;
#pragma unroll
    for (int d = 0; d < c; ++d) first = first && key[d] != key[c];
    if (first) {
      int n = 0;
#pragma unroll
      for (int d = c; d < 4; ++d) n += key[d] == key[c] ? 1 : 0;
      int at = atomicAdd(&cur[key[c]], n);
#pragma unroll
      for (int d = c; d < 4; ++d)
        if (key[d] == key[c]) slot[d] = at++;
    }
  }
}

// The four keys of the sample group whose eight coordinates start at `lc` (one
// 16-byte load for 16-bit locations, eight loads for float ones), at level lv.
template <typename TL>
__device__ inline void group_keys(const char* lc, const Level& lv, const LevelTiles& tl, int (&k)[4]) {
  using A = typename Elem<TL>::acc;
  A xy[8];
  if constexpr (sizeof(TL) == 2) {
    const u32x4_v w = *reinterpret_cast<const u32x4_v*>(lc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xy[2 * i] = Chan16<TL, 2>::lo(w[i]);
      xy[2 * i + 1] = Chan16<TL, 2>::hi(w[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) xy[i] = load_acc(reinterpret_cast<const TL*>(lc) + i);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) k[i] = sample_key<A>(xy[2 * i], xy[2 * i + 1], lv, tl);
}

template <int N> struct KeyWord;
template <> struct KeyWord<2> { using type = u32x2_v; };  // four 16-bit keys
template <> struct KeyWord<4> { using type = u32x4_v; };  // four 32-bit keys

// The bucketing passes for groups of 4 consecutive samples (q, s .. s + 3) of one
// query and level (L * P and P multiples of 4): one 16- or 32-byte location load and
// one query / level decode per group. Workgroup: kBucketThreads * SPT
// consecutive samples of one (b, h), thread t taking groups t, t + 256, ...
// The count pass publishes per-bucket counts as msda_bucket_kernel does and saves
// the four keys (16-bit when the keys fit, 0xffff / -1 for out of range) in the
// grad_value scratch, which nothing else uses before the sort ends; the place pass
// reads them back and hands out slots.
template <typename TL, bool PLACE, int KB, int SPT>
__global__ __launch_bounds__(kBucketThreads) void msda_bucket4_kernel(const Problem p, const BwdGeom bg,
                                                                      int* __restrict__ buckets,
                                                                      uint32_t* __restrict__ entries,
                                                                      int chunks_per_bh) {
  using A = typename Elem<TL>::acc;
  using Word = typename KeyWord<KB>::type;
  constexpr int kGroups = SPT / 4;  // groups per thread
  __shared__ int scan_sums[kBucketThreads / kWave];
  extern __shared__ __align__(16) unsigned char smem[];
  Level* levels = reinterpret_cast<Level*>(smem);
  LevelTiles* lt = reinterpret_cast<LevelTiles*>(smem + sizeof(Level) * size_t(p.L));
  const size_t head = ((sizeof(Level) + sizeof(LevelTiles)) * size_t(p.L) + 15) & ~size_t(15);
  int64_t* total = reinterpret_cast<int64_t*>(smem + head);
  int* hist = reinterpret_cast<int*>(smem + head + 16);
  bool overlap = false;
  const int64_t ntiles = load_tiles(p, bg, levels, lt, total, &overlap);
  const int64_t nkeys = 4 * ntiles;
  if (ntiles < 0 || nkeys > bg.keys_alloc) return;  // no bucketing: the owners scan
  // Overlapping levels: grad_value is zeroed for the owners' atomic adds, so the place
  // pass recomputes the keys instead of reading them back.
  const bool keep_keys = !overlap;
  if (!PLACE && overlap && p.zero_gv) zero_grad_value(p);
  const bool in_lds = nkeys <= bg.keys_lds;
  int group, h;
  if (!xcd_group_block(p.H, p.B * chunks_per_bh, &group, &h)) return;
  const int chunk = group % chunks_per_bh;
  const int b = group / chunks_per_bh;
  const int bh = b * p.H + h;
  const int LP = p.L * p.P;
  const int64_t nsamples = int64_t(p.Q) * LP;
  int* bucket_row = buckets + int64_t(bh) * nkeys;
  uint32_t* out = entries + int64_t(bh) * bg.region;
  Word* keys = reinterpret_cast<Word*>(p.grad_value) + int64_t(bh) * (bg.region / 4);
  const int64_t g0 = int64_t(chunk) * kBucketThreads * kGroups;  // first group of the chunk
  const int64_t ngroups = nsamples / 4;
  const uint32_t gpq = uint32_t(LP / 4);  // groups per query
  const char* loc_bh = reinterpret_cast<const char*>(p.loc) + (int64_t(b) * p.Q * p.H + h) * LP * 2 * int64_t(sizeof(TL));
  const uint32_t loc_q = uint32_t(p.H * LP * 2) * uint32_t(sizeof(TL));  // bytes per query

  // The four keys of group g (all -1 past the end).
  auto keys_of = [&](int64_t g, int (&k)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) k[i] = -1;
    if (g >= ngroups) return;
    const uint32_t g32 = uint32_t(g);
    const uint32_t q = fdiv(g32, bg.div_gpq), r = g32 - q * gpq;
    const int l = int(fdiv(r, bg.div_gpl));
    group_keys<TL>(loc_bh + (q * loc_q + r * uint32_t(8 * sizeof(TL))), levels[l], lt[l], k);
  };
  auto save = [&](int64_t g, const int (&k)[4]) __attribute__((always_inline)) {
    if (g >= ngroups || !keep_keys) return;
    Word w;
    if constexpr (KB == 2) {
      w[0] = (uint32_t(k[0]) & 0xffffu) | (uint32_t(k[1]) << 16);
      w[1] = (uint32_t(k[2]) & 0xffffu) | (uint32_t(k[3]) << 16);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = uint32_t(k[i]);
    }
    keys[g] = w;
  };
  auto restore = [&](int64_t g, int (&k)[4]) __attribute__((always_inline)) {
    if (!keep_keys) {
      keys_of(g, k);
      return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) k[i] = -1;
    if (g >= ngroups) return;
    const Word w = keys[g];
    if constexpr (KB == 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t v = (w[i >> 1] >> (16 * (i & 1))) & 0xffffu;
        k[i] = v == 0xffffu ? -1 : int(v);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) k[i] = int(w[i]);
    }
  };

  if (!in_lds) {
    // Too many buckets for LDS: one global atomic per sample.
    for (int i = 0; i < kGroups; ++i) {
      const int64_t g = g0 + int64_t(i) * kBucketThreads + threadIdx.x;
      int key[4];
      if constexpr (PLACE) {
        restore(g, key);
      } else {
        keys_of(g, key);
        save(g, key);
      }
      if constexpr (PLACE) {
        int slot[4];
        group_slots(key, bucket_row, slot);
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (key[c] >= 0) out[slot[c]] = uint32_t(4 * g + c);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (key[c] >= 0) atomicAdd(&bucket_row[key[c]], 1);
      }
    }
    return;
  }
  for (int64_t k = threadIdx.x; k < nkeys; k += kBucketThreads) hist[k] = 0;
  __syncthreads();
  if constexpr (!PLACE) {
#pragma unroll 2
    for (int i = 0; i < kGroups; ++i) {
      const int64_t g = g0 + int64_t(i) * kBucketThreads + threadIdx.x;
      int key[4];
      keys_of(g, key);
      save(g, key);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (key[c] >= 0) atomicAdd(&hist[key[c]], 1);
    }
    __syncthreads();
    if (chunked_sort(p, bg, nkeys)) {
      // Every count of this workgroup, zeros included, for the scan.
      int* row = chunk_counts(buckets, p, nkeys) + (int64_t(bh) * chunks_per_bh + chunk) * nkeys;
      for (int64_t k = threadIdx.x; k < nkeys; k += kBucketThreads) row[k] = hist[k];
    } else {
      for (int64_t k = threadIdx.x; k < nkeys; k += kBucketThreads) {
        const int c = hist[k];
        if (c > 0) atomicAdd(&bucket_row[k], c);
      }
    }
  } else {
    int key[kGroups][4];
#pragma unroll
    for (int i = 0; i < kGroups; ++i) restore(g0 + int64_t(i) * kBucketThreads + threadIdx.x, key[i]);
    if (chunked_sort(p, bg, nkeys)) {
      // This workgroup's offset in every bucket: the bucket's start (an exclusive
      // scan of the totals, here in LDS) plus the counts of the workgroups before it
      // (from the scan kernel). Workgroup 0 of each (b, h) writes the bucket ends.
      const int* tot = chunk_totals(buckets, p, bg, nkeys) + int64_t(bh) * nkeys;
      for (int64_t k = threadIdx.x; k < nkeys; k += kBucketThreads) hist[k] = tot[k];
      __syncthreads();
      int carry = 0;
      for (int64_t k0 = 0; k0 < nkeys; k0 += kBucketThreads) {
        const int64_t k = k0 + threadIdx.x;
        const int v = k < nkeys ? hist[k] : 0;
        int sum;
        const int ex = block_exclusive_scan(v, scan_sums, &sum);
        if (k < nkeys) {
          hist[k] = carry + ex;
          if (chunk == 0) bucket_row[k] = carry + ex + v;
        }
        carry += sum;
      }
      const int* row = chunk_counts(buckets, p, nkeys) + (int64_t(bh) * chunks_per_bh + chunk) * nkeys;
      for (int64_t k = threadIdx.x; k < nkeys; k += kBucketThreads) hist[k] += row[k];
    } else {
      // Counts again (from the saved keys), then this workgroup's range of every bucket.
#pragma unroll
      for (int i = 0; i < kGroups; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (key[i][c] >= 0) atomicAdd(&hist[key[i][c]], 1);
      __syncthreads();
      for (int64_t k = threadIdx.x; k < nkeys; k += kBucketThreads) {
        const int c = hist[k];
        if (c > 0) hist[k] = atomicAdd(&bucket_row[k], c);  // this workgroup's cursor in bucket k
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kGroups; ++i) {
      const int64_t g = g0 + int64_t(i) * kBucketThreads + threadIdx.x;
      int slot[4];
      group_slots(key[i], hist, slot);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (key[i][c] >= 0) out[slot[c]] = uint32_t(4 * g + c);
    }
  }
}

// The whole bucket sort of a small call in one launch: workgroup (b, h) counts its
// Q L P samples (in groups of 4, as msda_bucket4_kernel), scans the counts and places
// the samples, with the counters in LDS (or, when they do not fit there, in its own
// row of the scratch, which no other workgroup touches). No clear launch, no count
// rows and no second pass over the scratch: one launch where the general sort takes
// four, for calls whose (b, h) hold few samples. The bucket rows end up as the
// general sort leaves them (bucket ends), and workgroup 0 clears the matrix-core
// kernel's queue counters. Grid: B H workgroups.
constexpr int kSmallSortThreads = 1024;
constexpr int kSmallSortBatch = 4;  // groups per thread whose locations load together
template <typename TL>
__global__ __launch_bounds__(kSmallSortThreads) void msda_bucket_small_kernel(const Problem p, const BwdGeom bg,
                                                                             int* __restrict__ buckets,
                                                                             uint32_t* __restrict__ entries,
                                                                             int lds_keys) {
  __shared__ int scan_sums[kSmallSortThreads / kWave];
  extern __shared__ __align__(16) unsigned char smem[];
  Level* levels = reinterpret_cast<Level*>(smem);
  LevelTiles* lt = reinterpret_cast<LevelTiles*>(smem + sizeof(Level) * size_t(p.L));
  const size_t head = ((sizeof(Level) + sizeof(LevelTiles)) * size_t(p.L) + 15) & ~size_t(15);
  int64_t* total = reinterpret_cast<int64_t*>(smem + head);
  int* hist = reinterpret_cast<int*>(smem + head + 16);
  bool overlap = false;
  const int64_t ntiles = load_tiles(p, bg, levels, lt, total, &overlap);
  const int64_t nkeys = 4 * ntiles;
  if (ntiles < 0 || nkeys > bg.keys_alloc) return;  // no bucketing: the owners scan
  if (overlap && p.zero_gv) zero_grad_value(p);
  const int bh = int(blockIdx.x), b = bh / p.H, h = bh - b * p.H;
  const int T = int(blockDim.x), tid = int(threadIdx.x);
  int* bucket_row = buckets + int64_t(bh) * nkeys;
  int* cnt = nkeys <= lds_keys ? hist : bucket_row;
  for (int64_t k = tid; k < nkeys; k += T) cnt[k] = 0;
  if (bh == 0 && bg.sub_log2 > 0 && queue_fits(p, bg, nkeys))
    for (int i = tid; i < kQueueInts; i += T) buckets[int64_t(p.B) * p.H * nkeys + i] = 0;
  __syncthreads();

  const int LP = p.L * p.P;
  const int64_t ngroups = int64_t(p.Q) * LP / 4;
  const uint32_t gpq = uint32_t(LP / 4);
  const char* loc_bh = reinterpret_cast<const char*>(p.loc) + (int64_t(b) * p.Q * p.H + h) * LP * 2 * int64_t(sizeof(TL));
  const uint32_t loc_q = uint32_t(p.H * LP * 2) * uint32_t(sizeof(TL));
  auto keys_of = [&](int64_t g, int (&k)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) k[i] = -1;
    if (g >= ngroups) return;
    const uint32_t q = fdiv(uint32_t(g), bg.div_gpq), r = uint32_t(g) - q * gpq;
    const int l = int(fdiv(r, bg.div_gpl));
    group_keys<TL>(loc_bh + (q * loc_q + r * uint32_t(8 * sizeof(TL))), levels[l], lt[l], k);
  };
  const int64_t step = int64_t(T) * kSmallSortBatch;
  for (int64_t g0 = tid; g0 < ngroups; g0 += step) {
    int key[kSmallSortBatch][4];
#pragma unroll
    for (int i = 0; i < kSmallSortBatch; ++i) keys_of(g0 + int64_t(i) * T, key[i]);
#pragma unroll
    for (int i = 0; i < kSmallSortBatch; ++i)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (key[i][c] >= 0) atomicAdd(&cnt[key[i][c]], 1);
  }
  __syncthreads();
  // Counts to exclusive offsets (the place cursors); the bucket ends go to the row.
  // Counters in the row were added to at L2; they are read back from there.
  const bool in_lds = cnt != bucket_row;
  int carry = 0;
  for (int64_t k0 = 0; k0 < nkeys; k0 += T) {
    const int64_t k = k0 + tid;
    int v = 0;
    if (k < nkeys) v = in_lds ? cnt[k] : __hip_atomic_load(&cnt[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int sum;
    const int ex = block_exclusive_scan(v, scan_sums, &sum);
    if (k < nkeys) {
      cnt[k] = carry + ex;
      if (in_lds) bucket_row[k] = carry + ex + v;
    }
    carry += sum;
  }
  __syncthreads();
  uint32_t* out = entries + int64_t(bh) * bg.region;
  for (int64_t g0 = tid; g0 < ngroups; g0 += step) {
    int key[kSmallSortBatch][4];
#pragma unroll
    for (int i = 0; i < kSmallSortBatch; ++i) keys_of(g0 + int64_t(i) * T, key[i]);
#pragma unroll
    for (int i = 0; i < kSmallSortBatch; ++i) {
      int slot[4];
      group_slots(key[i], cnt, slot);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (key[i][c] >= 0) out[slot[c]] = uint32_t(4 * (g0 + int64_t(i) * T) + c);
    }
  }
}

// Counts to exclusive offsets. Unchunked: workgroup (b, h) < B H scans row (b, h).
// Chunked: thread (b, h, bucket) turns the bucket's per-workgroup counts into the
// counts of the workgroups before each (in place) and writes the bucket total; the
// place pass scans the totals. Workgroup 0 then also clears the matrix-core kernel's
// queue counters.
__global__ __launch_bounds__(256) void msda_bucket_scan_kernel(const Problem p, const BwdGeom bg,
                                                               int* __restrict__ buckets, int chunks_per_bh) {
  __shared__ Level levels_s[kMaxOrderedLevels];
  __shared__ LevelTiles lt_s[kMaxOrderedLevels];
  __shared__ int64_t total_s[2];
  __shared__ int wave_sums[256 / kWave];
  extern __shared__ __align__(16) unsigned char smem[];
  Level* levels = p.L <= kMaxOrderedLevels ? levels_s : reinterpret_cast<Level*>(smem);
  LevelTiles* lt = p.L <= kMaxOrderedLevels ? lt_s
                                             : reinterpret_cast<LevelTiles*>(smem + sizeof(Level) * size_t(p.L));
  const int64_t ntiles = load_tiles(p, bg, levels, lt, total_s);
  const int64_t nkeys = 4 * ntiles;
  if (ntiles < 0 || nkeys > bg.keys_alloc) return;
  const int64_t nbh = int64_t(p.B) * p.H;
  if (chunked_sort(p, bg, nkeys)) {
    if (blockIdx.x == 0)
      for (int i = threadIdx.x; i < kQueueInts; i += blockDim.x) buckets[nbh * nkeys + i] = 0;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < nbh * nkeys;
         i += int64_t(gridDim.x) * blockDim.x) {
      const int64_t bh = i / nkeys, k = i - bh * nkeys;
      int* cnt = chunk_counts(buckets, p, nkeys) + bh * chunks_per_bh * nkeys + k;
      constexpr int kBatch = 8;  // rows loaded together
      int run = 0;
      for (int c0 = 0; c0 < chunks_per_bh; c0 += kBatch) {
        int v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) v[u] = c0 + u < chunks_per_bh ? cnt[int64_t(c0 + u) * nkeys] : 0;
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          if (c0 + u < chunks_per_bh) cnt[int64_t(c0 + u) * nkeys] = run;
          run += v[u];
        }
      }
      chunk_totals(buckets, p, bg, nkeys)[i] = run;
    }
    return;
  }
  if (blockIdx.x >= nbh) return;
  int* row = buckets + int64_t(blockIdx.x) * nkeys;
  int carry = 0;
  for (int64_t k0 = 0; k0 < nkeys; k0 += blockDim.x) {
    const int64_t k = k0 + threadIdx.x;
    const int v = k < nkeys ? row[k] : 0;
    int sum;
    const int ex = block_exclusive_scan(v, wave_sums, &sum);
    if (k < nkeys) row[k] = carry + ex;
    carry += sum;
  }
}

// Clears the bucket counters: 4 * tiles ints per (b, h), with the tiles as the device
// plans them (the host knows only a bound).
__global__ __launch_bounds__(256) void msda_bucket_clear_kernel(const Problem p, const BwdGeom bg,
                                                                int* __restrict__ buckets) {
  __shared__ Level levels_s[kMaxOrderedLevels];
  __shared__ LevelTiles lt_s[kMaxOrderedLevels];
  __shared__ int64_t total_s[2];
  extern __shared__ __align__(16) unsigned char smem[];
  Level* levels = p.L <= kMaxOrderedLevels ? levels_s : reinterpret_cast<Level*>(smem);
  LevelTiles* lt = p.L <= kMaxOrderedLevels ? lt_s
                                             : reinterpret_cast<LevelTiles*>(smem + sizeof(Level) * size_t(p.L));
  const int64_t ntiles = load_tiles(p, bg, levels, lt, total_s);
  const int64_t nkeys = 4 * ntiles;
  if (ntiles < 0 || nkeys > bg.keys_alloc) return;
  if (chunked_sort(p, bg, nkeys)) return;  // the passes write every count; the scan clears the queues
  // The matrix-core grad_value keeps its work-queue counters right after the rows.
  const int64_t n = int64_t(p.B) * p.H * nkeys + (bg.sub_log2 > 0 && queue_fits(p, bg, nkeys) ? kQueueInts : 0);
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) buckets[i] = 0;
}

// The per-unit softmax statistics (see SoftStat), one lane per (b, q, h). A wave's 64
// units have contiguous logits: where they fit, the wave copies them to LDS with
// wide coalesced loads first (one load per lane and 16 bytes instead of one per
// logit at a 2- to 8-byte stride between lanes).
constexpr int kStatBytes = 64;  // logit bytes per unit staged through LDS, at most
template <typename T>
__global__ __launch_bounds__(256) void msda_softmax_stats_kernel(const Problem p, const BwdGeom bg,
                                                                  int* __restrict__ buckets) {
  using A = typename Elem<T>::acc;
  __shared__ Level levels_s[kMaxOrderedLevels];
  __shared__ LevelTiles lt_s[kMaxOrderedLevels];
  __shared__ int64_t total_s[2];
  extern __shared__ __align__(16) unsigned char smem[];
  Level* levels = p.L <= kMaxOrderedLevels ? levels_s : reinterpret_cast<Level*>(smem);
  LevelTiles* lt = p.L <= kMaxOrderedLevels ? lt_s
                                             : reinterpret_cast<LevelTiles*>(smem + sizeof(Level) * size_t(p.L));
  const int64_t ntiles = load_tiles(p, bg, levels, lt, total_s);
  const int64_t nkeys = 4 * ntiles;
  if (ntiles < 0 || nkeys > bg.keys_alloc || !softmax_stats_fit<A>(p, bg, nkeys, buckets)) return;
  SoftStat<A>* st = softmax_stats<A>(buckets, p, nkeys);
  __shared__ __align__(16) unsigned char lg_s[256 / kWave][kWave * kStatBytes];
  const int LP = p.L * p.P;
  const int ub = LP * int(sizeof(T));
  const bool staged = ub <= kStatBytes;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int64_t units = int64_t(p.B) * p.Q * p.H;
  const int64_t wave_step = int64_t(gridDim.x) * (blockDim.x / kWave) * kWave;
  for (int64_t u0 = (int64_t(blockIdx.x) * (blockDim.x / kWave) + wave) * kWave; u0 < units; u0 += wave_step) {
    const int64_t u = u0 + lane;
    const T* lg = reinterpret_cast<const T*>(p.attn) + u * LP;
    if (staged) {
      const int n = int(min<int64_t>(kWave, units - u0));
      copy_pieces(lg_s[wave], p.attn + u0 * ub, n * ub, p.attn_piece, lane);
      wave_lds_order();
      lg = reinterpret_cast<const T*>(lg_s[wave] + lane * ub);
    }
    if (u < units) {
      A mx = -INFINITY;
      for (int i = 0; i < LP; ++i) mx = fmax(mx, load_acc(lg + i));
      A sum(0);
      for (int i = 0; i < LP; ++i) sum += exp_acc(load_acc(lg + i) - mx);
      st[u] = SoftStat<A>{mx + log(sum)};
    }
    wave_lds_order();  // the lanes' reads come before the next copy
  }
}

// Zeroes grad_value[b, pos, :, :] at every position no valid level covers (every
// position when levels overlap); the tile owners write all the others.
template <typename T>
__global__ __launch_bounds__(256) void msda_gap_zero_kernel(const Problem p) {
  extern __shared__ __align__(16) unsigned char smem[];
  Level* levels = reinterpret_cast<Level*>(smem);
  if (threadIdx.x == 0) *overlap_flag() = 0;
  load_levels(p, levels);
  __syncthreads();
  overlap_flag_raise(levels, p.L);
  __syncthreads();
  // Overlapping levels: every position starts at zero for the atomic scatter.
  const bool overlap = *overlap_flag() != 0;
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= int64_t(p.B) * p.S) return;
  const int pos = int(idx % p.S);
  bool covered = false;
  for (int l = 0; l < p.L && !covered && !overlap; ++l) {
    const Level lv = levels[l];
    covered = lv.ok && pos >= lv.start && int64_t(pos) < int64_t(lv.start) + int64_t(lv.h) * lv.w;
  }
  if (covered) return;
  T* dst = reinterpret_cast<T*>(p.grad_value) + idx * p.H * p.D;
  for (int i = 0; i < p.H * p.D; ++i) store_elem(dst + i, typename Elem<T>::acc(0));
}

template <typename A> struct alignas(8) TileRec {
  A w;
  uint32_t off;  // byte offset of the record's staged grad_out row
};

// Raw (unconverted) loads for the prefetch, so that it does not wait for its data.
__device__ inline float to_acc(float v) { return v; }
__device__ inline double to_acc(double v) { return v; }
__device__ inline float to_acc(bf16_t v) { return __uint_as_float(uint32_t(v.bits) << 16); }
__device__ inline float to_acc(f16_t v) { return f16_bits(v.bits); }

template <typename TL> struct LocPair {
  TL x, y;
};

// One grad_out piece of CVR channels as a native vector type, so that arrays of
// them stay in VGPRs across the batch loop.
template <int BYTES> struct PieceOf;
template <> struct PieceOf<2> { using type = uint16_t; };
template <> struct PieceOf<4> { using type = uint32_t; };
template <> struct PieceOf<8> { using type = u32x2_v; };
template <> struct PieceOf<16> { using type = u32x4_v; };
template <typename T, int CVR> using Piece = typename PieceOf<Elem<T>::size * CVR>::type;

// How the owner kernel adds one corner record (weight w, staged grad_out piece g)
// into its CVR accumulators: acc[c] += w * g[c], with g widened to the accumulation
// type and w kept in it (fp32 for 16-bit values).
template <typename T, int CVR> struct OwnerAdd {
  using A = typename Elem<T>::acc;
  using Rec = TileRec<A>;
  static __device__ inline Rec make(A w, uint32_t off) { return Rec{w, off}; }
  static __device__ inline void add(A (&acc)[CVR], const Rec& r, const Piece<T, CVR>& pc) {
    A g[CVR];
    Chan<T, CVR>::from_raw(__builtin_bit_cast(Raw<Elem<T>::size * CVR>, pc), g);
#pragma unroll
    for (int c = 0; c < CVR; ++c) acc[c] = fma(r.w, g[c], acc[c]);
  }
};

// Exclusive prefix sum of n <= 4 * 64 counters by one wave (four per lane, DPP scan
// of the lane totals); writes start[0..n] and clears the counters.
__device__ inline void wave_scan_counts(int* cnt, int* start, int n) {
  const int lane = threadIdx.x & (kWave - 1);
  int v[4], sum = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = lane * 4 + j;
    v[j] = i < n ? cnt[i] : 0;
    sum += v[j];
  }
  const int inc = wave_inclusive_scan(sum);
  int run = inc - sum;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = lane * 4 + j;
    if (i < n) {
      start[i] = run;
      cnt[i] = 0;
    }
    run += v[j];
  }
  if (lane == kWave - 1) start[n] = inc;
}

// Orders the levels by expected records per tile (tile area / level area), heaviest
// first, so that the longest tiles start first, and numbers the tiles in that order:
// the tiles of order[i] have ranks rank_base[i] .. rank_base[i + 1] - 1. One thread.
__device__ inline void order_levels(const Problem& p, const Level* levels, const LevelTiles* lt,
                                    int* order, int* rank_base) {
  for (int i = 0; i < p.L; ++i) order[i] = i;
  if (p.L <= kMaxOrderedLevels) {
    for (int i = 0; i < p.L; ++i) {
      int best = i;
      for (int k = i + 1; k < p.L; ++k) {
        const int a = order[k], c = order[best];
        const int64_t ha = int64_t(levels[a].h) * levels[a].w, hc = int64_t(levels[c].h) * levels[c].w;
        const int64_t ta = int64_t(1) << (lt[a].lh + lt[a].lw), tc = int64_t(1) << (lt[c].lh + lt[c].lw);
        if (ta * hc > tc * ha) best = k;
      }
      const int tmp = order[i];
      order[i] = order[best];
      order[best] = tmp;
    }
  }
  int acc_tiles = 0;
  for (int i = 0; i < p.L; ++i) {
    rank_base[i] = acc_tiles;
    acc_tiles += lt[order[i]].ntx * lt[order[i]].nty;
  }
  rank_base[p.L] = acc_tiles;
}

// Owner-computes grad_value. Workgroup (slot, b, h) takes tiles slot, slot + nw, ...
// of (b, h) in descending order of expected records per tile. For each tile, batches
// of nb candidate samples:
//   A. thread t < nb turns candidate t into up to four corner records (position in
//      the tile, its sample slot, attention * bilinear weight) and ranks each record
//      within its position with an LDS integer atomic on the histogram;
//   B. one wave scans the histogram into each position's run (and clears it);
//   C. records move to run start + rank;
//   D. each thread walks the runs of the (position, channel group) items it owns
//      and accumulates weight * grad_out into fp32 registers, four records at a
//      time, from the batch's grad_out rows staged in LDS.
// Pipeline, three barriers per batch: after A each thread loads its sample of the
// next batch (location, weight) and its share of the next batch's grad_out rows
// (whose sample indices wait in LDS, `qnext`), plus its sample index two batches
// ahead; after D it moves them to registers and to the other of two grad_out row
// buffers. The loads are in flight during B, C and D.
template <typename T, typename TL, int CVR, bool SOFTMAX>
__global__ __launch_bounds__(kOwnerThreads) void msda_grad_value_kernel(
    const Problem p, const BwdGeom bg, const int* __restrict__ buckets,
    const uint32_t* __restrict__ entries, const int accumulate, const int after_mfma) {
  using A = typename Elem<T>::acc;
  using PieceT = Piece<T, CVR>;
  constexpr int ES = Elem<T>::size;
  constexpr int PB = ES * CVR;
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, wave = tid / kWave;
  const int G = bg.groups, nb = bg.nb, cap = bg.cap;
  const int LP = p.L * p.P;
  const uint32_t rstride = uint32_t(p.D) * ES + 16;  // padded rows: fewer bank conflicts

  // LDS layout; every offset is an integer added to smem, so accesses stay ds_*.
  size_t at = 0;
  Level* levels = reinterpret_cast<Level*>(smem + at);
  at += sizeof(Level) * size_t(p.L);
  LevelTiles* lt = reinterpret_cast<LevelTiles*>(smem + at);
  at += sizeof(LevelTiles) * size_t(p.L);
  int* order = reinterpret_cast<int*>(smem + at);  // levels, heaviest tiles first
  at += sizeof(int) * size_t(p.L);
  int* rank_base = reinterpret_cast<int*>(smem + at);  // first tile rank per ordered level
  at += sizeof(int) * size_t(p.L + 1);
  at = (at + 15) & ~size_t(15);
  int64_t* total = reinterpret_cast<int64_t*>(smem + at);
  at += 16;
  char* gtile = reinterpret_cast<char*>(smem + at);  // two buffers of nb grad_out rows
  const uint32_t gbuf = uint32_t(nb) * rstride;
  at += 2 * gbuf;
  using Add = OwnerAdd<T, CVR>;
  using Rec = typename Add::Rec;
  Rec* recs = reinterpret_cast<Rec*>(smem + at);
  at += sizeof(Rec) * size_t(4 * nb);
  uint32_t* qnext = reinterpret_cast<uint32_t*>(smem + at);  // next batch's sample indices
  at += sizeof(uint32_t) * size_t(nb);
  int* cnt = reinterpret_cast<int*>(smem + at);
  at += sizeof(int) * size_t(cap);
  int* start = reinterpret_cast<int*>(smem + at);  // cap + 1 entries

  const int64_t ntiles = load_tiles(p, bg, levels, lt, total);
  if (ntiles <= 0) return;
  if (after_mfma && queue_fits(p, bg, 4 * ntiles)) return;  // the matrix-core kernel did the work
  const bool bucketed = 4 * ntiles <= bg.keys_alloc;
  const SoftStat<A>* stats = !SOFTMAX ? nullptr
                             : p.stats ? reinterpret_cast<const SoftStat<A>*>(p.stats)
                             : bucketed && softmax_stats_fit<A>(p, bg, 4 * ntiles, buckets)
                                 ? softmax_stats<A>(const_cast<int*>(buckets), p, 4 * ntiles)
                                 : nullptr;
  if (tid == 0) {
    order_levels(p, levels, lt, order, rank_base);
    for (int i = 0; i < cap; ++i) cnt[i] = 0;
  }
  __syncthreads();

  // Groups (slot, b) in slot order, the heads of a group on one XCD: they run side by
  // side and share the cache lines of their queries' locations, weights and
  // grad_out rows. Groups are dealt round-robin to the XCDs, heaviest tiles first.
  int group, h;
  if (!xcd_group_block(p.H, bg.nw * p.B, &group, &h)) return;
  const int slot0 = group / p.B;
  const int b = group - slot0 * p.B;
  const int bh = b * p.H + h;
  const T* gout = reinterpret_cast<const T*>(p.grad_out);
  const T* attn_all = reinterpret_cast<const T*>(p.attn);
  const TL* loc_all = reinterpret_cast<const TL*>(p.loc);
  const uint32_t* ent = entries + int64_t(bh) * bg.region;
  const int* brow = buckets + int64_t(bh) * 4 * ntiles;
  const int64_t unit0 = int64_t(b) * p.Q * p.H + h;  // (b, q = 0, h)

  // Fixed per thread: the rows and channel groups of its staging pieces, and the
  // (position, channel group) items it owns.
  int prow[kOwnerChunks], pgrp[kOwnerChunks], ipos[kOwnerItems], igrp[kOwnerItems];
  uint32_t poff[kOwnerChunks];  // LDS byte offset of each staging piece in a row buffer
#pragma unroll
  for (int k = 0; k < kOwnerChunks; ++k) {
    const int u = tid + k * kOwnerThreads;
    prow[k] = u / G;
    pgrp[k] = u - prow[k] * G;
    poff[k] = uint32_t(prow[k]) * rstride + uint32_t(pgrp[k] * PB);
  }
#pragma unroll
  for (int k = 0; k < kOwnerItems; ++k) {
    const int u = tid + k * kOwnerThreads;
    ipos[k] = u / G;
    igrp[k] = u - ipos[k] * G;
  }

  for (int64_t trank = slot0; trank < ntiles; trank += bg.nw) {
    // The tile: level, rows [r0, r0 + th), columns [c0, c0 + tw), clipped to the level.
    int oi = 0;
    while (oi + 1 < p.L && rank_base[oi + 1] <= trank) ++oi;
    const int l = order[oi];
    const Level lv = levels[l];
    const LevelTiles tl = lt[l];
    const int tile = int(trank) - rank_base[oi];
    const int ty = tile / tl.ntx, tx = tile - ty * tl.ntx;
    const int r0 = ty << tl.lh, c0 = tx << tl.lw;
    const int r1 = min(r0 + (1 << tl.lh), lv.h), c1 = min(c0 + (1 << tl.lw), lv.w);
    const int npos = 1 << (tl.lh + tl.lw);  // positions past the level's edge stay empty

    // Candidate ranges: the tile's own sub-buckets and its neighbours' straddlers.
    uint32_t rs[4] = {0u, 0u, 0u, 0u}, rn[4] = {0u, 0u, 0u, 0u};
    if (bucketed) {
      auto range = [&](int k_first, int k_last, int i) __attribute__((always_inline)) {
        const uint32_t s0 = k_first > 0 ? uint32_t(brow[k_first - 1]) : 0u;
        rs[i] = s0;
        rn[i] = uint32_t(brow[k_last]) - s0;
      };
      const int kt = 4 * (tl.base + tile);
      range(kt, kt + 3, 0);
      if (tx > 0) range(kt - 4 + 1, kt - 4 + 2, 1);
      if (ty > 0) {
        const int ka = 4 * (tl.base + tile - tl.ntx);
        range(ka + 2, ka + 3, 2);
        if (tx > 0) range(ka - 4 + 2, ka - 4 + 2, 3);
      }
    } else {
      rn[0] = uint32_t(p.Q) * uint32_t(p.P);  // every sample of the level
    }
    const uint32_t n01 = rn[0] + rn[1], n012 = n01 + rn[2], ncand = n012 + rn[3];

    // The sample index (q * LP + s) of candidate c, or of a valid stand-in.
    auto entry_of = [&](uint32_t c) __attribute__((always_inline)) -> uint32_t {
      if (c >= ncand) c = 0;
      if (ncand == 0) return uint32_t(l * p.P);
      if (!bucketed) {
        const uint32_t q = fdiv(c, bg.div_p), pt = c - q * uint32_t(p.P);
        return q * uint32_t(LP) + uint32_t(l * p.P) + pt;
      }
      const uint32_t idx = c < rn[0] ? rs[0] + c
                           : c < n01 ? rs[1] + (c - rn[0])
                           : c < n012 ? rs[2] + (c - n01)
                                      : rs[3] + (c - n012);
      return ent[idx];
    };

    A accum[kOwnerItems][CVR];
#pragma unroll
    for (int k = 0; k < kOwnerItems; ++k)
#pragma unroll
      for (int c = 0; c < CVR; ++c) accum[k][c] = A(0);

    const uint32_t nbatch = (ncand + uint32_t(nb) - 1) / uint32_t(nb);
    const uint32_t own = uint32_t(tid < nb ? tid : 0);
    // Pipeline registers: `f_*` data of the next batch, `e_next` the own sample
    // index of the next batch, `e_after` that of the batch after it.
    LocPair<TL> f_loc{}, c_loc{};
    T f_attn{}, c_attn{};
    uint32_t f_own = 0, c_own = 0, e_next = 0, e_after = 0;
    PieceT f_piece[kOwnerChunks];
    auto issue = [&](uint32_t after_batch) __attribute__((always_inline)) {
      f_own = e_next;
      const uint32_t q = fdiv(f_own, bg.div_lp), s = f_own - q * uint32_t(LP);
      const int64_t unit = unit0 + int64_t(q) * p.H;
      f_loc = *reinterpret_cast<const LocPair<TL>*>(loc_all + (unit * LP + s) * 2);
      if constexpr (!SOFTMAX) f_attn = attn_all[unit * LP + s];
#pragma unroll
      for (int k = 0; k < kOwnerChunks; ++k) {
        const uint32_t e = qnext[prow[k] < nb ? prow[k] : 0];
        const uint32_t qr = fdiv(e, bg.div_lp);
        f_piece[k] = *reinterpret_cast<const PieceT*>(gout + (unit0 + int64_t(qr) * p.H) * p.D + pgrp[k] * CVR);
      }
      e_after = entry_of(after_batch * uint32_t(nb) + own);
    };
    // Move the loaded data of batch `batch` to registers and its grad_out rows to
    // their buffer; queue the indices of the batch after it.
    auto retire = [&](uint32_t batch) __attribute__((always_inline)) {
      c_loc = f_loc;
      c_attn = f_attn;
      c_own = f_own;
      char* buf = gtile + (batch & 1) * gbuf;
#pragma unroll
      for (int k = 0; k < kOwnerChunks; ++k)
        if (prow[k] < nb)
          *reinterpret_cast<PieceT*>(buf + poff[k]) = f_piece[k];
      if (tid < nb) qnext[tid] = e_after;
      e_next = e_after;
    };
    if (nbatch > 0) {
      // Prologue: the indices of batch 0 into qnext, then batch 0's data.
      e_next = entry_of(own);
      if (tid < nb) qnext[tid] = e_next;
      lds_barrier();
      issue(1);
      lds_barrier();
      retire(0);
    }
    lds_barrier();

    for (uint32_t bi = 0; bi < nbatch; ++bi) {
      const bool has = tid < nb && bi * uint32_t(nb) + uint32_t(tid) < ncand;
      // A. Records of the own sample.
      int rpos[4] = {0, 0, 0, 0}, rrank[4] = {0, 0, 0, 0};
      A rw[4] = {A(0), A(0), A(0), A(0)};
      bool rv[4] = {false, false, false, false};
      if (has) {
        const Geom<A> g = geometry<A>(to_acc(c_loc.x), to_acc(c_loc.y), lv, 0u, 1u);
        A a;
        if constexpr (SOFTMAX) {
          const uint32_t q = fdiv(c_own, bg.div_lp), s = c_own - q * uint32_t(LP);
          const int64_t u = unit0 + int64_t(q) * p.H;
          if (stats) {
            const SoftStat<A> st = stats[u];
            a = exp_acc(load_acc(attn_all + u * LP + s) - st.lse);
          } else {
            a = unit_weight<T, true>(attn_all + u * LP, LP, int(s));
          }
        } else {
          a = to_acc(c_attn);
        }
        const bool m[4] = {g.m00, g.m01, g.m10, g.m11};
        const A wb[4] = {g.w00, g.w01, g.w10, g.w11};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int cx = g.ix + (c & 1), cy = g.iy + (c >> 1);
          rv[c] = m[c] && cx >= c0 && cx < c1 && cy >= r0 && cy < r1;
          rpos[c] = ((cy - r0) << tl.lw) + (cx - c0);
          rw[c] = wb[c] * a;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (rv[c]) rrank[c] = atomicAdd(&cnt[rpos[c]], 1);
      }
      lds_barrier();
      issue(bi + 2);  // data of batch bi + 1, index of batch bi + 2
      // B. Run starts (one wave), counters cleared for the next batch.
      if (wave == 0) wave_scan_counts(cnt, start, npos);
      lds_barrier();
      // C. Place.
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (rv[c]) recs[start[rpos[c]] + rrank[c]] = Add::make(rw[c], uint32_t(tid) * uint32_t(rstride));
      lds_barrier();
      // D. Accumulate, four records at a time so that their LDS reads overlap.
      const char* cur = gtile + (bi & 1) * gbuf;
#pragma unroll
      for (int k = 0; k < kOwnerItems; ++k) {
        const int pos = ipos[k];
        if (pos < npos) {
          const char* gcol = cur + igrp[k] * PB;
          const int e1 = start[pos + 1];
          int r = start[pos];
          for (; r + 4 <= e1; r += 4) {
            Rec rec[4];
            PieceT pc[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) rec[u] = recs[r + u];
#pragma unroll
            for (int u = 0; u < 4; ++u) pc[u] = *reinterpret_cast<const PieceT*>(gcol + rec[u].off);
#pragma unroll
            for (int u = 0; u < 4; ++u) Add::add(accum[k], rec[u], pc[u]);
          }
          for (; r < e1; ++r) {
            const Rec rec = recs[r];
            Add::add(accum[k], rec, *reinterpret_cast<const PieceT*>(gcol + rec.off));
          }
        }
      }
      // Batch bi + 1 into the other buffer (last read by batch bi - 1, which every
      // wave finished before this batch's first barrier).
      retire(bi + 1);
    }
    lds_barrier();  // the last batch's reads are done before the next tile's prologue

    // The tile's positions: the only writer of these grad_value elements.
    const int64_t img = int64_t(b) * p.S * p.H * p.D;
#pragma unroll
    for (int k = 0; k < kOwnerItems; ++k) {
      const int pos = ipos[k];
      const int y = r0 + (pos >> tl.lw), x = c0 + (pos & ((1 << tl.lw) - 1));
      if (pos < npos && y < r1 && x < c1) {
        const int64_t gpos = int64_t(lv.start) + int64_t(y) * lv.w + x;
        char* dst = p.grad_value + (img + (gpos * p.H + h) * p.D + igrp[k] * CVR) * ES;
        if (accumulate) {
          A old[CVR];
          Chan<T, CVR>::load(dst, old);
#pragma unroll
          for (int c = 0; c < CVR; ++c) accum[k][c] += old[c];
        }
        Chan<T, CVR>::store(dst, accum[k]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// grad_value on the matrix cores: bf16, f16 and float values, D = 16, 32, 48 or 64.
//
// Tiles are 8 x 8 positions (sub_log2 = 3), bucketed as above, each made of four
// 4 x 4 sub-tiles. A (tile, head) task keeps the partial sums of its four sub-tiles
// (16 positions x D channels each) in the fp32 accumulators of the MFMA:
//   C_st[m, n] += sum_k W_st[m, k] * G[k, n]
// where G[k, :] is candidate k's grad_out row and W_st[m, k] the attention *
// bilinear weight of its corner at position m of sub-tile st (zero where it has
// none, so a sample adds exactly its corners in the tile). The candidates come in
// K-blocks of 64, one per lane; light tasks run one per wave, heavy ones split their
// K-blocks over the workgroup's four waves. Per K-block a wave stages the 64
// grad_out rows in its own LDS (row-major, bf16), and per K-step of 32 candidates
// scatters their corner weights into zeroed weight tiles and reads the operands
// back: A (position-major weight tiles) with ds_read_b128, B (grad_out, K-major)
// with two ds_read_b64_tr_b16 per 16 channels.
//
// Operands are split into two 16-bit parts, x = hi + lo + e: hi is x rounded to the
// operand type (nearest even) and lo the rest rounded again.
//   - bf16 values: v_mfma_f32_16x16x32_bf16, W (the fp32 attention * bilinear weight)
//     split into bf16 parts (|e| <= 2^-16 |W|: two weight tiles per sub-tile, W_hi
//     and W_lo), G exact in bf16.
//   - f16 values: v_mfma_f32_16x16x32_f16, W split into f16 parts (|e| <= 2^-22 |W|
//     while W_lo stays in f16's normal range, else |e| <= 2^-25), G exact in f16. W
//     never exceeds the f16 attention weight it scales, so W_hi cannot overflow.
//   - float values: v_mfma_f32_16x16x32_bf16 on bf16 parts of W and of G (two
//     staged row buffers, G_hi and G_lo).
//   - Per sub-tile, 16 channels and K-step the MFMAs add W_hi G_hi + W_lo G_hi, and
//     W_hi G_lo when G is split. Products are exact and sums fp32, so a product's
//     relative error is at most 2^-16 (bf16), 2^-22 (f16, normal range) and
//     3 * 2^-16 (float: the dropped W_lo G_lo and the two splits).
// Waves do not wait for each other inside a task; the loads of the next K-block (and
// the entries of the one after) are in flight while a K-block computes. A split
// task's four partial sums meet in LDS at its end and wave w writes sub-tile w.
//
// Operand layouts of v_mfma_f32_16x16x32 (wave64; lane l, g = l / 16, i = l % 16):
//   A: halves A[i][8 g .. 8 g + 7];  B: halves B[8 g .. 8 g + 7][i];
//   C: floats C[4 g .. 4 g + 3][i].
// ds_read_b64_tr_b16: inside each group of 16 lanes, lane i receives element i % 4
// of the 8-byte rows addressed by lanes i / 4 + 4 j, j = 0..3. Lane s addresses row
// 8 g + 4 t + s / 4 at channel 16 nb + 4 (s % 4), so lane i receives
// G[8 g + 4 t + j][16 nb + i]: half t of its B operand for channels 16 nb .. + 15.
//
// A non-finite grad_out channel reaches every position of the tiles its sample is a
// candidate of (0 * inf), not only the sample's corners. The low part of a
// non-finite value is zero, so an infinite product stays infinite.

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_v __attribute__((ext_vector_type(8)));
typedef float f32x4_v __attribute__((ext_vector_type(4)));
typedef short i16x4_v __attribute__((ext_vector_type(4)));

constexpr int kMfmaWaves = 4;     // waves per workgroup, splitting a tile's K-blocks
constexpr int kMfmaSubLog2 = 3;   // 8 x 8 position tiles of four 4 x 4 sub-tiles
constexpr int kMfmaK = 64;        // candidates per K-block: one per lane, two MFMA K-steps
constexpr int kMfmaKStep = 32;    // the MFMA's K
constexpr int kMfmaMaxNb = 4;     // 16-channel column blocks: D <= 64

// One 16 x 32 weight tile of 16-bit parts (16 positions, one K-step of candidates);
// a K-step has four sub-tiles of hi tiles, then four of lo tiles. A staged grad_out
// row holds 16 nb 16-bit channels.
constexpr int kMfmaWBytes = 16 * kMfmaKStep * 2;
constexpr int kMfmaLoTiles = 4 * kMfmaWBytes;  // offset of the lo tiles
constexpr int mfma_row_bytes(int nb) { return 16 * nb * 2; }
// The MFMA operand type of a value dtype: f16 for f16 values, bf16 otherwise.
template <typename T> constexpr bool mfma_f16_operands() { return std::is_same_v<T, f16_t>; }

template <bool F16>
__device__ inline f32x4_v mfma_16x16x32(const u32x4_v& a, const u32x4_v& b, f32x4_v c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_v, a), __builtin_bit_cast(f16x8_v, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_v, a), __builtin_bit_cast(bf16x8_v, b),
                                                   c, 0, 0, 0);
}

// The bf16 parts of x (see above); lo is zero for a non-finite x.
__device__ inline void split_bf16(float x, uint16_t* hi, uint16_t* lo) {
  const __bf16 h = static_cast<__bf16>(x);
  *hi = __builtin_bit_cast(uint16_t, h);
  const __bf16 r = static_cast<__bf16>(x - static_cast<float>(h));
  *lo = __builtin_isfinite(x) ? __builtin_bit_cast(uint16_t, r) : uint16_t(0);
}
// The f16 parts of x; lo is zero for a non-finite x.
__device__ inline void split_f16(float x, uint16_t* hi, uint16_t* lo) {
  const _Float16 h = static_cast<_Float16>(x);
  *hi = __builtin_bit_cast(uint16_t, h);
  const _Float16 r = static_cast<_Float16>(x - static_cast<float>(h));
  *lo = __builtin_isfinite(x) ? __builtin_bit_cast(uint16_t, r) : uint16_t(0);
}
// Two floats to packed (hi, lo) bf16 pairs, element 0 in the low halves.
__device__ inline void split_bf16_pair(float a, float b, uint32_t* hi, uint32_t* lo) {
  uint16_t ha, la, hb, lb;
  split_bf16(a, &ha, &la);
  split_bf16(b, &hb, &lb);
  *hi = uint32_t(ha) | (uint32_t(hb) << 16);
  *lo = uint32_t(la) | (uint32_t(lb) << 16);
}

// A wave-uniform value moved to a scalar register (it is the same in every lane).
__device__ inline int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ inline uint32_t uni(uint32_t v) { return uint32_t(__builtin_amdgcn_readfirstlane(int(v))); }

__device__ inline i16x4_v lds_read_tr16(const unsigned char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      reinterpret_cast<__attribute__((address_space(3))) i16x4_v*>(reinterpret_cast<uintptr_t>(p)));
}

// Per-wave LDS of the matrix-core kernel: the staged rows (one or two bf16 buffers)
// and the eight weight tiles during a tile, the wave's partial sums at its end.
size_t mfma_rows_bytes(int64_t D, bool split) {
  return size_t(kMfmaK) * size_t(mfma_row_bytes(int(D / 16))) * (split ? 2 : 1);
}
size_t mfma_wave_bytes(int64_t D, bool split) {
  const size_t work = mfma_rows_bytes(D, split) + 8 * size_t(kMfmaWBytes);
  const size_t partial = 4 * size_t(D / 16) * kWave * 16;
  return std::max(work, partial);
}

size_t mfma_head_bytes(int64_t L) {
  size_t at = (sizeof(Level) + sizeof(LevelTiles) + 2 * sizeof(int)) * size_t(L) + sizeof(int) * size_t(L + 1);
  at = (at + 15) & ~size_t(15);
  return at + 16;
}

size_t mfma_lds_bytes(int64_t L, int64_t D, bool split) {
  return mfma_head_bytes(L) + kMfmaWaves * mfma_wave_bytes(D, split);
}

// The candidates of one tile: ranges of the entry list (the tile's own
// sub-buckets, then its neighbours' straddlers); candidate c sits at entry
// c + off_k of the range k it falls in. `stand_in` is a valid sample index for
// candidates past the end.
struct CandRanges {
  uint32_t n0, n01, n012, ncand;
  uint32_t off0, off1, off2, off3;
  uint32_t stand_in;
};

__device__ inline CandRanges tile_candidates(const int* __restrict__ brow, const LevelTiles& tl, int tile,
                                             int tx, int ty, uint32_t stand_in) {
  uint32_t rs[4] = {0u, 0u, 0u, 0u}, rn[4] = {0u, 0u, 0u, 0u};
  const int kt = 4 * (tl.base + tile);
  const uint32_t s0 = kt > 0 ? uint32_t(brow[kt - 1]) : 0u;
  rs[0] = s0;
  rn[0] = uint32_t(brow[kt + 3]) - s0;
  if (tx > 0) {  // left neighbour, sub-buckets 1-2
    rs[1] = uint32_t(brow[kt - 4]);
    rn[1] = uint32_t(brow[kt - 2]) - rs[1];
  }
  if (ty > 0) {
    const int ka = 4 * (tl.base + tile - tl.ntx);
    rs[2] = uint32_t(brow[ka + 1]);  // tile above, sub-buckets 2-3
    rn[2] = uint32_t(brow[ka + 3]) - rs[2];
    if (tx > 0) {  // above-left, sub-bucket 2
      rs[3] = uint32_t(brow[ka - 4 + 1]);
      rn[3] = uint32_t(brow[ka - 4 + 2]) - rs[3];
    }
  }
  CandRanges r;
  r.n0 = uni(rn[0]);
  r.n01 = uni(rn[0] + rn[1]);
  r.n012 = uni(r.n01 + rn[2]);
  r.ncand = uni(r.n012 + rn[3]);
  r.off0 = uni(rs[0]);
  r.off1 = uni(rs[1] - r.n0);
  r.off2 = uni(rs[2] - r.n01);
  r.off3 = uni(rs[3] - r.n012);
  r.stand_in = stand_in;
  return r;
}

// The sample index of candidate c (candidate 0 past the end); needs ncand > 0.
__device__ inline uint32_t cand_entry(const uint32_t* __restrict__ ent, const CandRanges r, uint32_t c) {
  c = c < r.ncand ? c : 0u;
  uint32_t off = r.off3;
  off = c < r.n012 ? r.off2 : off;
  off = c < r.n01 ? r.off1 : off;
  off = c < r.n0 ? r.off0 : off;
  return ent[c + off];
}

// One K-block's loads for one lane: its candidate's location and weight (MfmaMeta,
// loaded a block ahead), and its share of the block's grad_out rows (MfmaRows: flat
// 16-byte piece lane + 64 j of the 64 rows, loaded half a block ahead, as soon as
// the previous block has staged its rows).
template <typename T, typename TL> struct MfmaMeta {
  LocPair<TL> loc;
  T attn;              // the weight, or with softmax the logit
  SoftStat<float> st;  // softmax: the unit's statistics (when stats are kept)
};
template <int NP> struct MfmaRows {
  u32x4_v piece[NP];
};
// 16-byte pieces of one grad_out row of 16 NB channels (each lane loads as many).
template <typename T, int NB> constexpr int mfma_pieces() { return NB * int(sizeof(T)); }

// Per-tile constants of the matrix-core kernel (all wave-uniform).
struct MfmaTile {
  const char* loc;   // locations of (b, q = 0, h)
  const char* attn;  // weights of (b, q = 0, h)
  const char* gout;  // grad_out row of (b, q = 0, h)
  uint32_t loc_q, attn_q, gout_q;  // bytes per query step
  int r0, c0, r1, c1;              // tile rows [r0, r1), columns [c0, c1)
  int nst;                         // sub-tiles the tile has: 4 (8 x 8), or 1 (4 x 4)
  uint32_t ncand;
  FastDiv div_lp;
  int LP;
  const SoftStat<float>* stats;  // softmax statistics of (b, q = 0, h), stride H per query; or null
  int H;
};

template <typename T, typename TL, bool SOFTMAX>
__device__ inline void mfma_load_meta(const MfmaTile& t, uint32_t e, MfmaMeta<T, TL>& d) {
  const uint32_t q = fdiv(e, t.div_lp), s = e - q * uint32_t(t.LP);
  d.loc = *reinterpret_cast<const LocPair<TL>*>(t.loc + (__umul24(q, t.loc_q) + s * uint32_t(2 * sizeof(TL))));
  if (!SOFTMAX || t.stats) d.attn = *reinterpret_cast<const T*>(t.attn + (__umul24(q, t.attn_q) + s * uint32_t(sizeof(T))));
  if constexpr (SOFTMAX)
    if (t.stats) d.st = t.stats[__umul24(q, uint32_t(t.H))];
}

template <typename T, int NB>
__device__ inline void mfma_load_rows(const MfmaTile& t, uint32_t e, int lane, MfmaRows<mfma_pieces<T, NB>()>& d) {
  constexpr int kPieces = mfma_pieces<T, NB>();  // 16-byte pieces per grad_out row
  const uint32_t q = fdiv(e, t.div_lp);
#pragma unroll
  for (int j = 0; j < kPieces; ++j) {
    const int f = lane + kWave * j, row = f / kPieces, pc = f - row * kPieces;
    const uint32_t qr = uint32_t(__shfl(int(q), row));
    d.piece[j] = *reinterpret_cast<const u32x4_v*>(t.gout + (__umul24(qr, t.gout_q) + uint32_t(pc * 16)));
  }
}

// One K-block of one wave, in two parts. Part A: the candidate's corners (as LDS
// byte offsets of their weights in the hi weight tiles, -1 outside the tile, and the
// weights' 16-bit parts), and the block's 64 grad_out rows into LDS as 16-bit
// operands (hi and lo buffers when split), after which the row registers are free for the next
// block's loads. Part B: per MFMA K-step (the candidates of lanes 0-31, then 32-63)
// scatter the corner weights into the weight tiles, run the sub-tiles' MFMAs, and
// clear the scattered entries again. The tiles are zeroed once (mfma_zero_tiles) and
// are all zeros between K-steps: clearing at most eight 2-byte entries per lane costs
// far less LDS bandwidth than zeroing the 8 KB of tiles per K-step. A wave's LDS
// instructions execute in order, so the clears land after the operand reads.
struct MfmaCorners {
  int o[4];
  uint16_t hi[4], lo[4];
};

// A staged 16-byte piece of a grad_out row: copied (bf16, f16), or split into bf16
// hi and lo parts (float: 4 channels, 8 bytes each).
template <typename T>
__device__ inline void mfma_stage_piece(const u32x4_v& v, unsigned char* hi, unsigned char* lo) {
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<u32x4_v*>(hi) = v;
  } else {
    u32x2_v h, l;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      uint32_t hw, lw;
      split_bf16_pair(__uint_as_float(v[2 * i]), __uint_as_float(v[2 * i + 1]), &hw, &lw);
      h[i] = hw;
      l[i] = lw;
    }
    *reinterpret_cast<u32x2_v*>(hi) = h;
    *reinterpret_cast<u32x2_v*>(lo) = l;
  }
}

template <typename T, typename TL, int NB, bool SOFTMAX>
__device__ inline MfmaCorners mfma_kblock_a(const MfmaTile& t, const Level& lv, uint32_t kb, uint32_t e,
                                            const MfmaMeta<T, TL>& d, const MfmaRows<mfma_pieces<T, NB>()>& rows,
                                            int lane, unsigned char* gst) {
  constexpr int ES = int(sizeof(T));
  constexpr int kPieces = mfma_pieces<T, NB>();
  constexpr int kRowBytes = mfma_row_bytes(NB);
  constexpr int kStagedPiece = 16 * 2 / ES;  // staged bytes a 16-byte piece becomes
  constexpr size_t kLoRows = size_t(kMfmaK) * kRowBytes;
  const int kc = lane & (kMfmaKStep - 1);
  const uint32_t c = kb * kMfmaK + uint32_t(lane);
  MfmaCorners cr;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    cr.o[k] = -1;
    cr.hi[k] = cr.lo[k] = 0;
  }
  if (c < t.ncand) {
    const Geom<float> g = geometry<float>(to_acc(d.loc.x), to_acc(d.loc.y), lv, 0u, 1u);
    float a;
    if constexpr (SOFTMAX) {
      if (t.stats) {
        a = exp_acc(to_acc(d.attn) - d.st.lse);
      } else {
        const uint32_t q = fdiv(e, t.div_lp), s = e - q * uint32_t(t.LP);
        a = unit_weight<T, true>(reinterpret_cast<const T*>(t.attn + __umul24(q, t.attn_q)), t.LP, int(s));
      }
    } else {
      a = to_acc(d.attn);
    }
    const bool m[4] = {g.m00, g.m01, g.m10, g.m11};
    const float wb[4] = {g.w00, g.w01, g.w10, g.w11};
    const int y0 = g.iy - t.r0, x0 = g.ix - t.c0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int y = y0 + (k >> 1), x = x0 + (k & 1);
      // Position (y, x) of the tile: sub-tile (y / 4) * 2 + x / 4, row (y % 4) * 4 + x % 4
      // of its position-major [16][32] weight tile.
      if (m[k] && y >= 0 && x >= 0 && t.r0 + y < t.r1 && t.c0 + x < t.c1) {
        const int pos = (y & 3) * 4 + (x & 3);
        cr.o[k] = ((y >> 2) * 2 + (x >> 2)) * kMfmaWBytes + pos * (2 * kMfmaKStep) + kc * 2;
        if constexpr (mfma_f16_operands<T>())
          split_f16(wb[k] * a, &cr.hi[k], &cr.lo[k]);
        else
          split_bf16(wb[k] * a, &cr.hi[k], &cr.lo[k]);
      }
    }
  }
  wave_lds_order();  // after the previous K-block's operand reads
  const u32x4_v zero = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < kPieces; ++j) {
    const int f = lane + kWave * j, row = f / kPieces, pc = f - row * kPieces;
    const bool ok = kb * kMfmaK + uint32_t(row) < t.ncand;  // past the end: zero rows
    unsigned char* dst = gst + row * kRowBytes + pc * kStagedPiece;
    mfma_stage_piece<T>(ok ? rows.piece[j] : zero, dst, dst + kLoRows);
  }
  return cr;
}

// TAIL: a tile's last K-blocks, whose second K-step may hold no candidate.
template <typename T, int NB, int NST, bool TAIL = false>
__device__ inline void mfma_kblock_b(const MfmaCorners& cr, int lane, const unsigned char* gst, unsigned char* wt,
                                     f32x4_v (&acc)[4][NB], int ksteps = 2) {
  constexpr bool kSplit = sizeof(T) == 4;
  constexpr bool kF16 = mfma_f16_operands<T>();
  constexpr int kRowBytes = mfma_row_bytes(NB);
  constexpr size_t kLoRows = size_t(kMfmaK) * kRowBytes;
  const int half = lane >> 5;
  const int g16 = lane >> 4, i16 = lane & 15;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    if constexpr (TAIL)
      if (ks >= ksteps) break;  // wave-uniform: the K-step holds no candidate
    wave_lds_order();
    if (half == ks) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (cr.o[k] >= 0) {
          *reinterpret_cast<uint16_t*>(wt + cr.o[k]) = cr.hi[k];
          *reinterpret_cast<uint16_t*>(wt + kMfmaLoTiles + cr.o[k]) = cr.lo[k];
        }
    }
    wave_lds_order();
    u32x4_v bh[NB], bl[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const unsigned char* src =
          gst + (kMfmaKStep * ks + 8 * g16 + i16 / 4) * kRowBytes + (16 * nb + 4 * (i16 & 3)) * 2;
      bh[nb] = __builtin_bit_cast(u32x4_v, __builtin_shufflevector(lds_read_tr16(src), lds_read_tr16(src + 4 * kRowBytes),
                                                                    0, 1, 2, 3, 4, 5, 6, 7));
      if constexpr (kSplit)
        bl[nb] = __builtin_bit_cast(u32x4_v, __builtin_shufflevector(lds_read_tr16(src + kLoRows),
                                                                      lds_read_tr16(src + kLoRows + 4 * kRowBytes),
                                                                      0, 1, 2, 3, 4, 5, 6, 7));
    }
    const int aoff = i16 * (2 * kMfmaKStep) + g16 * 16;
#pragma unroll
    for (int st = 0; st < NST; ++st) {  // NST = 1: a 4 x 4 tile is sub-tile 0
      const u32x4_v ah = *reinterpret_cast<const u32x4_v*>(wt + st * kMfmaWBytes + aoff);
      const u32x4_v al = *reinterpret_cast<const u32x4_v*>(wt + kMfmaLoTiles + st * kMfmaWBytes + aoff);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if constexpr (kSplit) acc[st][nb] = mfma_16x16x32<false>(ah, bl[nb], acc[st][nb]);
        acc[st][nb] = mfma_16x16x32<kF16>(al, bh[nb], acc[st][nb]);
        acc[st][nb] = mfma_16x16x32<kF16>(ah, bh[nb], acc[st][nb]);
      }
    }
    wave_lds_order();
    if (half == ks) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (cr.o[k] >= 0) {
          *reinterpret_cast<uint16_t*>(wt + cr.o[k]) = 0;
          *reinterpret_cast<uint16_t*>(wt + kMfmaLoTiles + cr.o[k]) = 0;
        }
    }
  }
}

// Zeroes a wave's eight weight tiles (once per wave, and again after its LDS served
// for partial sums).
__device__ inline void mfma_zero_tiles(unsigned char* wt, int lane) {
  const u32x4_v zero = {0u, 0u, 0u, 0u};
  wave_lds_order();
#pragma unroll
  for (int z = 0; z < 8 * kMfmaWBytes / (kWave * 16); ++z)
    *reinterpret_cast<u32x4_v*>(wt + (z * kWave + lane) * 16) = zero;
  wave_lds_order();
}

// K-steps of K-block kb that hold candidates (the rest would add zeros).
__device__ inline int mfma_ksteps(const MfmaTile& t, uint32_t kb) {
  return t.ncand > kb * kMfmaK + kMfmaKStep ? 2 : 1;
}

// The K-blocks kb0, kb0 + kbstep, ... of one tile into acc (zeroed here). Block j's
// entries are loaded two blocks ahead, its locations and weights one block ahead
// (two register sets in turn) and its grad_out rows as soon as block j - 1 has
// staged its own, each before the loads of later blocks, so that a wait for one
// never waits for younger loads. The main loop issues its loads unconditionally
// (an entry past the end reads candidate 0), so that the compiler's wait counts
// stay exact; the last one or two blocks run after it.
template <typename T, typename TL, int NB, bool SOFTMAX, int NST>
__device__ inline void mfma_tile_kblocks(const MfmaTile& t, const Level& lv, const CandRanges& cr,
                                         const uint32_t* __restrict__ ent, int kb0, int kbstep, int lane,
                                         unsigned char* gst, unsigned char* wt, f32x4_v (&acc)[4][NB]) {
#pragma unroll
  for (int st = 0; st < 4; ++st)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[st][j] = f32x4_v{0.f, 0.f, 0.f, 0.f};
  const uint32_t nkb = (cr.ncand + kMfmaK - 1) / kMfmaK;
  const uint32_t mine = nkb > uint32_t(kb0) ? (nkb - uint32_t(kb0) + uint32_t(kbstep) - 1) / uint32_t(kbstep) : 0u;
  const uint32_t step = uint32_t(kbstep) * kMfmaK;
  uint32_t cand = uint32_t(kb0) * kMfmaK + uint32_t(lane);  // this lane's candidate in block j
  MfmaMeta<T, TL> ma, mb;
  MfmaRows<mfma_pieces<T, NB>()> rows;
  uint32_t ea = 0, eb = 0, j = 0;
  if (mine > 0) {
    ea = cand_entry(ent, cr, cand);
    eb = cand_entry(ent, cr, cand + step);
    mfma_load_meta<T, TL, SOFTMAX>(t, ea, ma);
    mfma_load_rows<T, NB>(t, ea, lane, rows);
  }
  for (; j + 2 < mine; j += 2) {
    const uint32_t kb = uint32_t(kb0) + j * uint32_t(kbstep);
    const uint32_t e2 = cand_entry(ent, cr, cand + 2 * step);
    mfma_load_meta<T, TL, SOFTMAX>(t, eb, mb);
    const auto c0 = mfma_kblock_a<T, TL, NB, SOFTMAX>(t, lv, kb, ea, ma, rows, lane, gst);
    mfma_load_rows<T, NB>(t, eb, lane, rows);
    mfma_kblock_b<T, NB, NST>(c0, lane, gst, wt, acc);
    const uint32_t e3 = cand_entry(ent, cr, cand + 3 * step);
    mfma_load_meta<T, TL, SOFTMAX>(t, e2, ma);
    const auto c1 = mfma_kblock_a<T, TL, NB, SOFTMAX>(t, lv, kb + uint32_t(kbstep), eb, mb, rows, lane, gst);
    mfma_load_rows<T, NB>(t, e2, lane, rows);
    mfma_kblock_b<T, NB, NST>(c1, lane, gst, wt, acc);
    ea = e2;
    eb = e3;
    cand += 2 * step;
  }
  if (j < mine) {
    const uint32_t kb = uint32_t(kb0) + j * uint32_t(kbstep);
    const bool two = j + 1 < mine;
    if (two) mfma_load_meta<T, TL, SOFTMAX>(t, eb, mb);
    const auto c0 = mfma_kblock_a<T, TL, NB, SOFTMAX>(t, lv, kb, ea, ma, rows, lane, gst);
    if (two) mfma_load_rows<T, NB>(t, eb, lane, rows);
    mfma_kblock_b<T, NB, NST, true>(c0, lane, gst, wt, acc, mfma_ksteps(t, kb));
    if (two) {
      const auto c1 = mfma_kblock_a<T, TL, NB, SOFTMAX>(t, lv, kb + uint32_t(kbstep), eb, mb, rows, lane, gst);
      mfma_kblock_b<T, NB, NST, true>(c1, lane, gst, wt, acc, mfma_ksteps(t, kb + uint32_t(kbstep)));
    }
  }
}

// Writes sub-tile st of a tile from the MFMA layout: lane l holds C[4 g + r][16 nb + i]
// = position (r0 + 4 (st / 2) + g, c0 + 4 (st % 2) + r), channel 16 nb + i. The tile
// owns these grad_value elements: one plain store each (a load-add-store with
// `accumulate`).
template <typename T, int NB>
__device__ inline void mfma_store_subtile(const Problem& p, const Level& lv, const MfmaTile& t, int b, int h,
                                          int st, const f32x4_v (&c)[NB], int g16, int i16, int accumulate,
                                          T* gv, bool add = false) {
  constexpr int D = 16 * NB;
  // add (wave-uniform): overlapping levels. Tiles of two levels own the shared
  // positions, so each adds its fp32 sums with one atomic per element (float) or per
  // channel pair (16-bit: the even lane adds its pair, the odd lane's value taken with
  // a DPP move that every lane runs, before the per-lane bounds test): one rounding
  // for the sum and one for the add per level, where a 16-bit atomic scatter rounds
  // once per contribution.
  const int y = t.r0 + 4 * (st >> 1) + g16;
  const bool yok = y < t.r1;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int x = t.c0 + 4 * (st & 1) + r;
    const bool ok = yok && x < t.c1;
    const int64_t pos = int64_t(b) * p.S + lv.start + int64_t(y) * lv.w + x;
    T* dst = gv + (pos * p.H + h) * D + i16;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (add) {
        if constexpr (std::is_same_v<T, float>) {
          if (ok) unsafeAtomicAdd(dst + 16 * nb, c[nb][r]);
        } else {
          const float pair = quad_perm<kQuadXor1>(c[nb][r]);
          if (ok && (i16 & 1) == 0) {
            if constexpr (std::is_same_v<T, bf16_t>) {
              const bf16x2_v v2 = {static_cast<__bf16>(c[nb][r]), static_cast<__bf16>(pair)};
              __builtin_amdgcn_global_atomic_fadd_v2bf16(reinterpret_cast<bf16x2_v*>(dst + 16 * nb), v2);
            } else {
              const f16x2_v v2 = {static_cast<_Float16>(c[nb][r]), static_cast<_Float16>(pair)};
              __builtin_amdgcn_global_atomic_fadd_v2f16(reinterpret_cast<f16x2_v*>(dst + 16 * nb), v2);
            }
          }
        }
      } else if (ok) {
        float v = c[nb][r];
        if (accumulate) v += load_acc(dst + 16 * nb);
        store_elem(dst + 16 * nb, v);
      }
    }
  }
}

// Workgroups per CU the register budget of the matrix-core kernel allows (float
// values prefetch twice the row bytes of 16-bit ones).
constexpr int mfma_blocks_per_cu(int nb, int es) {
  return es == 4 ? (nb == 1 ? 3 : 2) : (nb == 1 ? 4 : nb == 2 ? 3 : 2);
}

constexpr int kMfmaMaxRegions = 8;   // regions per axis at most
constexpr int kMfmaTable = 1024;      // entries of a queue's prefix table at most
constexpr int kMfmaMaxChunk = 8;      // tasks a workgroup takes from its queue at once, at most

// Region (x, y) of Morton (Z-order) index z: x takes the even bits, y the odd ones,
// so consecutive indices stay in compact 2D blocks.
__device__ inline void morton_decode(int z, int* x, int* y) {
  int rx = 0, ry = 0;
  for (int bit = 0; bit < 8; ++bit) {
    rx |= ((z >> (2 * bit)) & 1) << bit;
    ry |= ((z >> (2 * bit + 1)) & 1) << bit;
  }
  *x = rx;
  *y = ry;
}

// The first tile column (or row) of region r of n regions across a level `extent`
// positions wide with `ntiles` tiles of side S: tile t, centred at position
// S t + S / 2, lies in region floor((S t + S / 2) n / extent).
__device__ inline int region_first_tile(int r, int n, int extent, int ntiles, int S) {
  if (r >= n) return ntiles;
  const int64_t num = int64_t(r) * extent - int64_t(S / 2) * n;
  if (num <= 0) return 0;
  const int64_t den = int64_t(S) * n;
  return int(std::min<int64_t>(ntiles, (num + den - 1) / den));
}

// Work distribution: a persistent grid with one work queue per XCD (a counter in
// the scratch after the bucket counters; workgroup w serves queue w % 8, the XCD the
// dispatcher deals it to). The image is cut into R x R regions in normalized
// coordinates, and a tile of any level belongs to the region of its centre: the
// tiles of one region at all levels gather nearly the same queries, because a
// query samples every level at the same normalized place. Queue x holds the x-th
// eighth of the (b, region) pairs, regions in Morton order; per pair the tasks
// (tile, h) run level by level,
// heaviest tiles first, heads fastest. So an XCD's workgroups share one compact
// neighbourhood of queries in their L2 at a time, and a workgroup that finishes
// early takes the next task of its queue. A small LDS table of prefix counts per
// (pair, level) maps a queue position to its task. When the table would not fit,
// queue x holds the x-th eighth of each level's tasks (b, tile, h) in raster order.
template <typename T, typename TL, int NB, bool SOFTMAX>
__global__ __launch_bounds__(kWave * kMfmaWaves, mfma_blocks_per_cu(NB, int(sizeof(T)))) void msda_grad_value_mfma_kernel(
    const Problem p, const BwdGeom bg, int* __restrict__ buckets,
    const uint32_t* __restrict__ entries, const int accumulate, const int table_cap) {
  constexpr int D = 16 * NB;
  constexpr int ES = int(sizeof(T));
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int wave_sums[kMfmaWaves];
  __shared__ int grid_s[2];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int LP = p.L * p.P;

  size_t at = 0;
  Level* levels = reinterpret_cast<Level*>(smem + at);
  at += sizeof(Level) * size_t(p.L);
  LevelTiles* lt = reinterpret_cast<LevelTiles*>(smem + at);
  at += sizeof(LevelTiles) * size_t(p.L);
  int* order = reinterpret_cast<int*>(smem + at);
  at += sizeof(int) * size_t(p.L);
  int* rank_base = reinterpret_cast<int*>(smem + at);
  at += sizeof(int) * size_t(p.L + 1);
  int* csz = reinterpret_cast<int*>(smem + at);  // tasks per chunk of each ordered level
  at += sizeof(int) * size_t(p.L);
  at = (at + 15) & ~size_t(15);
  int64_t* total = reinterpret_cast<int64_t*>(smem + at);  // [0]: tiles, [1]: the fetched task
  at += 16;
  constexpr bool kSplit = sizeof(T) == 4;
  constexpr size_t kRowsBytes = size_t(kMfmaK) * size_t(mfma_row_bytes(NB)) * (kSplit ? 2 : 1);
  constexpr size_t kWaveBytes = std::max(kRowsBytes + 8 * size_t(kMfmaWBytes), size_t(4 * NB * kWave * 16));
  unsigned char* region0 = smem + at;
  unsigned char* gst = region0 + size_t(wave) * kWaveBytes;  // grad_out rows (hi, then lo)
  unsigned char* wt = gst + kRowsBytes;                      // eight weight tiles (hi, then lo)
  // Per (pair, level) of this XCD's queue: prefix count of chunks, and tasks.
  int* table = reinterpret_cast<int*>(region0 + size_t(kMfmaWaves) * kWaveBytes);
  int* ntab = table + table_cap + 1;

  bool overlap;
  const int64_t ntiles = load_tiles(p, bg, levels, lt, total, &overlap);
  // Overlapping levels on the owners: the count pass zeroed grad_value, and the owners add.
  const bool add = p.sort_overlap && overlap;
  if (!accumulate && !add) {
    // grad_value at positions no valid level covers is zero (the tiles own all the
    // others, so this never meets their stores); when levels overlap and the owners
    // stand aside, every position starts at zero for the atomic scatter.
    const int64_t n = int64_t(p.B) * p.S;
    for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + tid; idx < n; idx += int64_t(gridDim.x) * blockDim.x) {
      const int pos = int(idx % p.S);
      bool covered = false;
      for (int l = 0; l < p.L && !covered && !overlap; ++l) {
        const Level lv = levels[l];
        covered = lv.ok && pos >= lv.start && int64_t(pos) < int64_t(lv.start) + int64_t(lv.h) * lv.w;
      }
      if (!covered) {
        T* dst = reinterpret_cast<T*>(p.grad_value) + idx * p.H * D;
        for (int i = 0; i < p.H * D; ++i) store_elem(dst + i, 0.f);
      }
    }
  }
  if (ntiles <= 0 || !queue_fits(p, bg, 4 * ntiles)) return;  // the VALU owner kernel runs instead
  const bool stats_ok = SOFTMAX && (p.stats || softmax_stats_fit<float>(p, bg, 4 * ntiles, buckets));
  if (tid == 0) {
    order_levels(p, levels, lt, order, rank_base);
    // R x R regions, R the power of two nearest the finest level's tile count, at most
    // kMfmaMaxRegions.
    int mt = 1;
    for (int i = 0; i < p.L; ++i) mt = max(mt, max(lt[i].ntx, lt[i].nty));
    int r = 1;
    while (r < kMfmaMaxRegions && 2 * r <= mt) r *= 2;
    grid_s[0] = r;
    // A tile's expected work goes as (tile area) / (level area): chunks of the level
    // with the heaviest tiles hold one task, a level whose tiles expect k times less
    // work min(k, kMfmaMaxChunk) tasks.
    int64_t amin = 0, tmin = 1;  // the heaviest tiles' level area over their tile area: amin / tmin
    for (int i = 0; i < p.L; ++i) {
      const int64_t area = int64_t(levels[i].h) * levels[i].w, tarea = int64_t(1) << (lt[i].lh + lt[i].lw);
      if (levels[i].ok && (amin == 0 || area * tmin < amin * tarea)) {
        amin = area;
        tmin = tarea;
      }
    }
    for (int i = 0; i < p.L; ++i) {
      const int l = order[i];
      const int64_t area = int64_t(levels[l].h) * levels[l].w, tarea = int64_t(1) << (lt[l].lh + lt[l].lw);
      const int64_t k = amin > 0 ? (area * tmin) / (amin * tarea) : 1;
      csz[i] = int(std::max<int64_t>(1, std::min<int64_t>(kMfmaMaxChunk, k)));
    }
  }
  __syncthreads();

  const int xcd = int(blockIdx.x) % kXcds;
  int* queue = reinterpret_cast<int*>(
                   (reinterpret_cast<uintptr_t>(buckets + int64_t(p.B) * p.H * 4 * ntiles) + 4 * kQueueLine - 1) &
                   ~uintptr_t(4 * kQueueLine - 1)) +
               xcd * kQueueLine;
  const int64_t per_tile = int64_t(p.B) * p.H;
  const int R = grid_s[0];  // regions per axis, a power of two; visited in Morton order
  const int64_t npairs = int64_t(p.B) * R * R;
  const int64_t pa = xcd * npairs / kXcds, pb = (xcd + 1) * npairs / kXcds;
  const int64_t nentries = (pb - pa) * p.L;
  // The same choice on every XCD (the queues' pair counts differ by one when npairs
  // is not a multiple of 8): either every queue holds (pair, level) entries or every
  // queue holds an eighth of each level's tasks, never a mix of the two.
  const bool regional = (npairs + kXcds - 1) / kXcds * p.L <= table_cap;
  int64_t queue_len = 0;
  if (regional) {
    // Chunks per (pair, level), then their exclusive prefix sums: four entries a thread.
    int cnt[4], sum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = tid * 4 + j;
      cnt[j] = 0;
      if (i < nentries) {
        const int64_t pair = pa + i / p.L;
        const int l = order[i % p.L];
        int rx, ry;
        morton_decode(int(pair % (R * R)), &rx, &ry);
        const Level lv = levels[l];
        const LevelTiles tl = lt[l];
        const int nx = region_first_tile(rx + 1, R, lv.w, tl.ntx, 1 << tl.lw) - region_first_tile(rx, R, lv.w, tl.ntx, 1 << tl.lw);
        const int ny = region_first_tile(ry + 1, R, lv.h, tl.nty, 1 << tl.lh) - region_first_tile(ry, R, lv.h, tl.nty, 1 << tl.lh);
        ntab[i] = nx * ny * p.H;
        cnt[j] = (ntab[i] + csz[i % p.L] - 1) / csz[i % p.L];
      }
      sum += cnt[j];
    }
    int all;
    int run = block_exclusive_scan(sum, wave_sums, &all);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = tid * 4 + j;
      if (i <= nentries) table[i] = run;
      run += cnt[j];
    }
    queue_len = all;
  } else {
    for (int oi = 0; oi < p.L; ++oi) {
      const int64_t n = int64_t(rank_base[oi + 1] - rank_base[oi]) * per_tile;
      queue_len += (xcd + 1) * n / kXcds - xcd * n / kXcds;
    }
  }
  __syncthreads();
  const int g16 = lane >> 4, i16 = lane & 15;
  mfma_zero_tiles(wt, lane);

  // Thread 0 takes chunks from the queue and publishes them in chunk_s: entry i
  // (-1: the queue is empty) and its tasks [first, last). Regional chunks of light
  // levels (chunk size >= 4) run one task per wave with no partial sums to merge;
  // the others run one task at a time, its K-blocks split over the four waves.
  __shared__ int chunk_s[3];
  for (;;) {
    if (tid == 0) {
      int ci = -1, first = 0, last = 0;
      const int64_t c = atomicAdd(queue, 1);
      if (c < queue_len) {
        if (regional) {
          int lo = 0, hi = int(nentries) - 1;  // the last entry whose prefix is <= c
          while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (table[mid] <= c) lo = mid; else hi = mid - 1;
          }
          const int cs = csz[lo % p.L];
          ci = lo;
          first = int(c - table[lo]) * cs;
          last = min(first + cs, ntab[lo]);
        } else {
          ci = 0;
          first = int(c);
          last = first + 1;
        }
      }
      chunk_s[0] = ci;
      chunk_s[1] = first;
      chunk_s[2] = last;
    }
    __syncthreads();
    const int ci = chunk_s[0], first = chunk_s[1], last = chunk_s[2];
    if (ci < 0) break;  // uniform: every thread read the same value
    const bool per_wave = regional && csz[ci % p.L] >= kMfmaWaves;
    const int step = per_wave ? kMfmaWaves : 1;
    for (int base = first; base < last; base += step) {
      const int local = per_wave ? base + wave : base;
      if (local >= last) continue;  // only in the per-wave mode, where waves do not sync
      // The task: level l, image b, head h, tile.
      int l, b, h, tile;
      if (regional) {
        const int64_t pair = pa + ci / p.L;
        l = order[ci % p.L];
        b = int(pair / (R * R));
        int rx, ry;
        morton_decode(int(pair % (R * R)), &rx, &ry);
        const Level lvr = levels[l];
        const LevelTiles tlr = lt[l];
        const int tx0 = region_first_tile(rx, R, lvr.w, tlr.ntx, 1 << tlr.lw);
        const int nx = region_first_tile(rx + 1, R, lvr.w, tlr.ntx, 1 << tlr.lw) - tx0;
        const int ty0 = region_first_tile(ry, R, lvr.h, tlr.nty, 1 << tlr.lh);
        h = local % p.H;
        const int rest = local / p.H;
        tile = (ty0 + rest / nx) * tlr.ntx + tx0 + rest % nx;
      } else {
        int64_t k = local;
        // The queue's k-th task: level order[oi], task t of that level.
        int oi = 0;
        int64_t tl_task = 0;
        for (; oi < p.L; ++oi) {
          const int64_t n = int64_t(rank_base[oi + 1] - rank_base[oi]) * per_tile;
          const int64_t lo = xcd * n / kXcds, len = (xcd + 1) * n / kXcds - lo;
          if (k < len) {
            tl_task = lo + k;
            break;
          }
          k -= len;
        }
        l = order[oi];
        const LevelTiles tlr = lt[l];
        const int ntl = tlr.ntx * tlr.nty;
        h = int(tl_task % p.H);
        const int64_t rest = tl_task / p.H;
        tile = int(rest % ntl);
        b = int(rest / ntl);
      }
      l = uni(l);
      b = uni(b);
      h = uni(h);
      tile = uni(tile);
      Level lv = levels[l];
      lv = Level{uni(lv.h), uni(lv.w), uni(lv.start), uni(lv.ok)};
      LevelTiles tl = lt[l];
      tl = LevelTiles{uni(tl.lh), uni(tl.lw), uni(tl.ntx), uni(tl.nty), uni(tl.base)};
      const int ty = tile / tl.ntx, tx = tile - ty * tl.ntx;
      const int bh = b * p.H + h;
      const uint32_t* ent = entries + int64_t(bh) * bg.region;
      const CandRanges cr = tile_candidates(buckets + int64_t(bh) * 4 * ntiles, tl, tile, tx, ty, uint32_t(l * p.P));
      const int64_t unit0 = int64_t(b) * p.Q * p.H + h;  // (b, q = 0, h)
      MfmaTile t;
      t.loc = p.loc + unit0 * LP * 2 * int64_t(sizeof(TL));
      t.attn = p.attn + unit0 * LP * ES;
      t.gout = p.grad_out + unit0 * D * ES;
      t.loc_q = uint32_t(p.H * LP * 2) * uint32_t(sizeof(TL));
      t.attn_q = uint32_t(p.H * LP * ES);
      t.gout_q = uint32_t(p.H * D * ES);
      t.r0 = ty << tl.lh;
      t.c0 = tx << tl.lw;
      t.r1 = min(t.r0 + (1 << tl.lh), lv.h);
      t.c1 = min(t.c0 + (1 << tl.lw), lv.w);
      t.nst = tl.lw < kMfmaSubLog2 ? 1 : 4;  // a 4 x 4 tile is sub-tile 0 alone
      t.ncand = cr.ncand;
      t.div_lp = bg.div_lp;
      t.LP = LP;
      t.H = p.H;
      t.stats = SOFTMAX && stats_ok ? (p.stats ? reinterpret_cast<const SoftStat<float>*>(p.stats)
                                               : softmax_stats<float>(buckets, p, 4 * ntiles)) + unit0
                                    : nullptr;

      f32x4_v acc[4][NB];
      // All K-blocks (per-wave mode), or K-blocks wave, wave + 4, ...
      if (t.nst == 1)  // wave-uniform: a 4 x 4 tile runs one sub-tile's MFMAs
        mfma_tile_kblocks<T, TL, NB, SOFTMAX, 1>(t, lv, cr, ent, per_wave ? 0 : wave, per_wave ? 1 : kMfmaWaves,
                                                 lane, gst, wt, acc);
      else
        mfma_tile_kblocks<T, TL, NB, SOFTMAX, 4>(t, lv, cr, ent, per_wave ? 0 : wave, per_wave ? 1 : kMfmaWaves,
                                                 lane, gst, wt, acc);

      T* gv = reinterpret_cast<T*>(p.grad_value);
      if (per_wave) {
        // Lane l holds C[4 g + r][16 nb + i] of sub-tile st: position
        // (r0 + 4 (st / 2) + g, c0 + 4 (st % 2) + r), channel 16 nb + i.
#pragma unroll
        for (int st = 0; st < 4; ++st)
          mfma_store_subtile<T, NB>(p, lv, t, b, h, st, acc[st], g16, i16, accumulate, gv, add);
        continue;
      }
      // Partial sums meet in LDS (each wave's own region, which only it used so
      // far): wave w adds the four waves' sums of sub-tile w.
      {
        u32x4_v* out = reinterpret_cast<u32x4_v*>(gst);
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) out[(st * NB + nb) * kWave + lane] = __builtin_bit_cast(u32x4_v, acc[st][nb]);
      }
      __syncthreads();
      f32x4_v sum[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        sum[nb] = f32x4_v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < kMfmaWaves; ++w)
          sum[nb] += __builtin_bit_cast(
              f32x4_v, reinterpret_cast<const u32x4_v*>(region0 + size_t(w) * kWaveBytes)[(wave * NB + nb) * kWave + lane]);
      }
      mfma_store_subtile<T, NB>(p, lv, t, b, h, wave, sum, g16, i16, accumulate, gv, add);
      __syncthreads();  // the partial sums are read before the next tile reuses the LDS
      mfma_zero_tiles(wt, lane);
    }
    __syncthreads();  // every wave is done with the chunk before the next one is published
  }
}

// Samples of a unit whose corner loads grad_sample issues together.
constexpr int kSampleBatch = 2;

// G_c = <grad_out, value at corner c> for the staged samples s .. s + N - 1 of the
// lane's unit, summed over the unit's lanes, into the samples' slots. The corner
// loads of all N samples go out before the first dot product (the cross-lane sums
// keep the compiler from unrolling a loop over samples). For two samples in units of
// 4 or 8 float lanes the eight sums are reduce-scattered (unit_reduce_scatter8) and
// each lane stores the ones it ends with; otherwise every lane forms all the sums and
// the lane that staged a sample stores its four.
template <typename T, int CV, int N>
__device__ inline void corner_dots(const LaneMap& m, Staged<typename Elem<T>::acc>* wst, int s, bool lane_ok,
                                   const char* img, uint32_t row_bytes, uint32_t lane_bytes,
                                   const typename Chan<T, CV>::R& g) {
  using A = typename Elem<T>::acc;
  using R = typename Chan<T, CV>::R;
  Staged<A> st[N];
#pragma unroll
  for (int n = 0; n < N; ++n) st[n] = wst[(s + n) * m.uw_count + m.uw];
  A G[N][4];
#pragma unroll
  for (int n = 0; n < N; ++n)
#pragma unroll
    for (int c = 0; c < 4; ++c) G[n][c] = A(0);
  if (lane_ok) {
    R v[N][4];
#pragma unroll
    for (int n = 0; n < N; ++n)
#pragma unroll
      for (int c = 0; c < 4; ++c) v[n][c] = *reinterpret_cast<const R*>(row_at(img, st[n].off[c], row_bytes, lane_bytes));
#pragma unroll
    for (int n = 0; n < N; ++n)
#pragma unroll
      for (int c = 0; c < 4; ++c) G[n][c] = Chan<T, CV>::dot(g, v[n][c], G[n][c]);
  }
  if constexpr (N == 2 && __is_same(A, float)) {
    if (m.lh == 4 || m.lh == 8) {
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = G[i >> 2][i & 3];
      unit_reduce_scatter8(v, m.lh, m.t);
      if (m.unit_ok) {
        // Lane t holds sum t (lh = 8) or sums 2 t, 2 t + 1 (lh = 4); sum i is sample
        // s + i / 4, corner i % 4.
        const int i0 = m.lh == 8 ? m.t : 2 * m.t;
        wst[(s + (i0 >> 2)) * m.uw_count + m.uw].w[i0 & 3] = v[0];
        if (m.lh == 4) wst[(s + (i0 >> 2)) * m.uw_count + m.uw].w[(i0 & 3) + 1] = v[1];
      }
      return;
    }
  }
#pragma unroll
  for (int n = 0; n < N; ++n)
#pragma unroll
    for (int c = 0; c < 4; ++c) G[n][c] = unit_sum(G[n][c], m.lh);
#pragma unroll
  for (int n = 0; n < N; ++n) {
    if (m.unit_ok && m.t == ((s + n) & (m.lh - 1))) {
      Staged<A>* slot = wst + (s + n) * m.uw_count + m.uw;
#pragma unroll
      for (int c = 0; c < 4; ++c) slot->w[c] = G[n][c];
    }
  }
}

// A location gradient pair: one 4-byte store for 16-bit locations (grad_loc is
// 4-byte aligned), else one store per coordinate.
template <typename TL, typename A>
__device__ inline void store_loc_pair(TL* p, A x, A y) {
  if constexpr (sizeof(TL) == 2) {
    *reinterpret_cast<uint32_t*>(p) = Chan16<TL, 2>::pack(x, y);
  } else {
    store_elem(p, x);
    store_elem(p + 1, y);
  }
}

// Location and weight gradients, sample-parallel, laid out like the forward.
template <typename T, typename TL, int CV, bool SOFTMAX>
__global__ __launch_bounds__(kWave * kMaxWavesPerBlock) void msda_grad_sample_kernel(const Problem p) {
  using A = typename Elem<T>::acc;
  constexpr int ES = Elem<T>::size;
  extern __shared__ __align__(16) unsigned char smem[];
  Level* levels = reinterpret_cast<Level*>(smem);
  const LaneMap m = map_lane(p);
  const int LP = p.L * p.P;
  Staged<A>* wst = reinterpret_cast<Staged<A>*>(smem + sizeof(Level) * p.L) +
                   m.wave * m.uw_count * LP;
  const size_t raw_at =
      (sizeof(Level) * p.L + sizeof(Staged<A>) * (blockDim.x / kWave) * m.uw_count * LP + 15) & ~size_t(15);
  const UnitRaw raw = copy_unit_records<T, TL>(p, m, smem + raw_at);

  if (threadIdx.x == 0) *overlap_flag() = 0;
  load_levels(p, levels);
  __syncthreads();
  overlap_flag_raise(levels, p.L);
  A smax, sinv, ssum = A(1);
  stage_samples<T, TL, SOFTMAX>(p, m, levels, raw, wst, smax, sinv, &ssum);
  if constexpr (SOFTMAX)  // the unit's log-sum-exp for the grad_value kernel, as msda_softmax_stats_kernel's
    if (p.stats && m.unit_ok && m.t == 0) reinterpret_cast<SoftStat<A>*>(p.stats)[m.gunit] = SoftStat<A>{smax + log(ssum)};
  __syncthreads();
  // grad_value by atomics: asked for, or levels overlap where the owners stand aside
  // (the sort and the owners then only zeroed grad_value).
  const bool scatter = (*overlap_flag() != 0 && !p.sort_overlap) || p.atomic_gv;

  // Gather the corners and form G_c; the lane that staged sample s keeps its G_c
  // in the sample's slot.
  using R = typename Chan<T, CV>::R;
  const bool lane_ok = m.unit_ok && m.t * CV < p.D;
  const int64_t img_bytes = int64_t(m.b) * p.S * p.H * p.D * ES;
  const char* img = p.value + img_bytes;
  char* gv_img = scatter ? p.grad_value + img_bytes : nullptr;
  const uint32_t row_bytes = uint32_t(p.D * ES), lane_bytes = uint32_t(m.t * CV * ES);
  R g{};
  if (lane_ok) g = *reinterpret_cast<const R*>(p.grad_out + (m.gunit * p.D + m.t * CV) * ES);
  if (gv_img != nullptr && lane_ok) {
    // Each lane adds weight * grad_out into its channels of every corner with a
    // non-zero weight, with global atomics (before the dots overwrite the weights).
    A gw[CV];
    Chan<T, CV>::from_raw(g, gw);
    for (int s = 0; s < LP; ++s) {
      const Staged<A> st = wst[s * m.uw_count + m.uw];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (st.w[c] != A(0))
          atomic_add_channels<T, CV>(row_at(gv_img, st.off[c], row_bytes, lane_bytes), st.w[c], gw);
    }
  }
  int s = 0;
  for (; s + kSampleBatch <= LP; s += kSampleBatch)
    corner_dots<T, CV, kSampleBatch>(m, wst, s, lane_ok, img, row_bytes, lane_bytes, g);
  for (; s < LP; ++s) corner_dots<T, CV, 1>(m, wst, s, lane_ok, img, row_bytes, lane_bytes, g);
  wave_lds_order();  // other lanes of the unit stored some of a sample's sums

  // Per-sample location and weight gradients by the lane that staged the sample.
  const TL* loc = reinterpret_cast<const TL*>(raw.loc);
  const T* attn = reinterpret_cast<const T*>(raw.attn);
  TL* gloc = reinterpret_cast<TL*>(p.grad_loc) + m.gunit * LP * 2;
  T* gattn = reinterpret_cast<T*>(p.grad_attn) + m.gunit * LP;
  A dot(0);
  if (m.unit_ok) {
    for (int s = m.t; s < LP; s += m.lh) {
      const Level lv = levels[s / p.P];
      const Geom<A> ge = geometry<A>(load_acc(loc + 2 * s), load_acc(loc + 2 * s + 1), lv, 0u, 1u);
      A a = load_acc(attn + s);
      if constexpr (SOFTMAX) a = exp_acc(a - smax) * sinv;
      Staged<A>* slot = wst + s * m.uw_count + m.uw;
      A gx, gy, gpv;
      sample_grads<A>(ge, a, lv, slot->w[0], slot->w[1], slot->w[2], slot->w[3], &gx, &gy, &gpv);
      store_loc_pair(gloc + 2 * s, gx, gy);
      if constexpr (SOFTMAX) {
        dot += a * gpv;
        slot->w[0] = gpv;
      } else {
        store_elem(gattn + s, gpv);
      }
    }
  }
  if constexpr (SOFTMAX) {
    dot = unit_sum(dot, m.lh);
    if (m.unit_ok) {
      for (int s = m.t; s < LP; s += m.lh) {
        const A a = exp_acc(load_acc(attn + s) - smax) * sinv;
        const A gpv = wst[s * m.uw_count + m.uw].w[0];
        store_elem(gattn + s, a * (gpv - dot));
      }
    }
  }
}

// Zero-fill for empty calls: a plain kernel (not hipMemsetAsync), so a caller may
// capture the call in a HIP graph.
__global__ __launch_bounds__(256) void zero_fill_kernel(char* p, int64_t bytes) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const int64_t head = int64_t((16 - (a & 15)) & 15) < bytes ? int64_t((16 - (a & 15)) & 15) : bytes;
  const int64_t body = (bytes - head) / 16;
  uint4* q = reinterpret_cast<uint4*>(p + head);
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < body; i += stride)
    q[i] = make_uint4(0, 0, 0, 0);
  if (blockIdx.x == 0) {
    const int64_t tail0 = head + body * 16;
    for (int64_t i = threadIdx.x; i < head; i += blockDim.x) p[i] = 0;
    for (int64_t i = tail0 + threadIdx.x; i < bytes; i += blockDim.x) p[i] = 0;
  }
}

// ---------------------------------------------------------------------------
// Host side.

thread_local char g_last_error[1024] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int elem_size(int dtype) {
  switch (dtype) {
    case MSDA_F32: return 4;
    case MSDA_F16: return 2;
    case MSDA_BF16: return 2;
    case MSDA_F64: return 8;
    default: return 0;
  }
}

const char* dtype_name(int dtype) {
  switch (dtype) {
    case MSDA_F32: return "float32";
    case MSDA_F16: return "float16";
    case MSDA_BF16: return "bfloat16";
    case MSDA_F64: return "float64";
    default: return "unknown";
  }
}

struct Plan {
  int cv, lh_log2, waves, units_per_block, blocks_per_batch;
  int64_t num_blocks;
  size_t lds;
};

bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

// Choose the channel width, the unit width and the workgroup size.
int make_plan(int dtype, int64_t B, int64_t S, int64_t H, int64_t D, int64_t Q, int64_t L,
              int64_t P, bool backward, const void* const* vec_ptrs, int n_vec, Plan* plan, int loc_es) {
  const int es = elem_size(dtype);
  if (es == 0) return fail(MSDA_ERR_INVALID, "msda: unknown value dtype code %d", dtype);
  if (B < 0 || S < 0 || H < 0 || D < 0 || Q < 0 || L < 0 || P < 0)
    return fail(MSDA_ERR_INVALID, "msda: negative size (B=%lld S=%lld H=%lld D=%lld Q=%lld L=%lld P=%lld)",
                (long long)B, (long long)S, (long long)H, (long long)D, (long long)Q,
                (long long)L, (long long)P);
  if (H == 0 || D == 0 || L == 0 || P == 0)
    return fail(MSDA_ERR_INVALID, "msda: heads, channels, levels and points must be positive");
  const int64_t kInt32 = 2147483647;
  if (S * H * D >= kInt32)
    return fail(MSDA_ERR_UNSUPPORTED,
                "msda: one batch image of value holds %lld elements; the kernels index an image's "
                "rows with 32-bit offsets and take at most 2^31 - 1 elements",
                (long long)(S * H * D));
  if (Q * H >= kInt32 || L * P > 4096 || B >= kInt32)
    return fail(MSDA_ERR_UNSUPPORTED, "msda: queries * heads, batch or levels * points too large");
  // Channels per lane: the widest power of two that divides D, fits a 16-byte
  // access and keeps every channel pointer aligned to that access.
  int cv = 16 / es;
  while (cv > 1) {
    bool ok = D % cv == 0;
    for (int i = 0; i < n_vec && ok; ++i) ok = aligned(vec_ptrs[i], cv * es);
    if (ok) break;
    cv >>= 1;
  }
  const int64_t lanes = D / cv;
  if (lanes > kWave)
    return fail(MSDA_ERR_UNSUPPORTED,
                "msda: %lld channels per head need %lld lanes of %d channels; at most %d",
                (long long)D, (long long)lanes, cv, kWave);
  int lh_log2 = 0;
  while ((1 << lh_log2) < lanes) ++lh_log2;
  const size_t staged = dtype == MSDA_F64 ? sizeof(Staged<double>) : sizeof(Staged<float>);
  const size_t levels_bytes = sizeof(Level) * size_t(L);
  // Per wave: the staged records of its units, and the LDS copy of their locations
  // and weights. When one wave's units do not fit, a unit takes more lanes (the
  // lanes past the channels stage samples and idle in the gathers), so a wave holds
  // fewer units.
  auto lds_for = [&](int lhl, int w) {
    const int u = kWave >> lhl;
    const size_t per_wave = size_t(u) * size_t(L * P) * staged;
    const size_t raw_wave = size_t(unit_raw_bytes(u, int(L * P), loc_es, es));
    return ((levels_bytes + per_wave * w + 15) & ~size_t(15)) + raw_wave * w;
  };
  while (lh_log2 < 6 && lds_for(lh_log2, 1) > kMaxLds) ++lh_log2;
  const int uw = kWave >> lh_log2;
  auto lds_of = [&](int w) { return lds_for(lh_log2, w); };
  if (lds_of(1) > kMaxLds)
    return fail(MSDA_ERR_UNSUPPORTED,
                "msda: %lld samples per (query, head) do not fit the %zu-byte LDS staging of one "
                "wave (%zu bytes needed)",
                (long long)(L * P), kMaxLds, lds_of(1));
  const int64_t units = Q * H;
  int waves = kMaxWavesPerBlock;
  // Fewer waves per workgroup when the grid would leave CUs idle or LDS is short.
  while (waves > 1) {
    const int64_t blocks = B * ((units + int64_t(waves) * uw - 1) / (int64_t(waves) * uw));
    if (lds_of(waves) <= kMaxLds && blocks >= 2048) break;
    waves >>= 1;
  }
  plan->cv = cv;
  plan->lh_log2 = lh_log2;
  plan->waves = waves;
  plan->units_per_block = waves * uw;
  plan->blocks_per_batch = int((units + plan->units_per_block - 1) / plan->units_per_block);
  plan->num_blocks = B * plan->blocks_per_batch;
  plan->lds = lds_of(waves);
  if (plan->num_blocks * kWave * waves >= (int64_t(1) << 32) || plan->num_blocks >= kInt32)
    return fail(MSDA_ERR_UNSUPPORTED, "msda: launch grid too large (%lld workgroups)",
                (long long)plan->num_blocks);
  return MSDA_OK;
}

// Dispatch on (value dtype, location dtype, channels per lane): f is a generic
// lambda taking <T, TL, CV> template arguments.
template <typename T, typename TL, typename F>
hipError_t dispatch_cv(int cv, F& f) {
  constexpr int kMaxCv = 16 / Elem<T>::size;
  switch (cv) {
    case 1: return f.template operator()<T, TL, 1>();
    case 2: return f.template operator()<T, TL, 2>();
    case 4:
      if constexpr (kMaxCv >= 4) return f.template operator()<T, TL, 4>();
      break;
    case 8:
      if constexpr (kMaxCv >= 8) return f.template operator()<T, TL, 8>();
      break;
  }
  return hipErrorInvalidValue;
}

template <typename F>
hipError_t dispatch(int dtype, bool loc_f32, int cv, F&& f) {
  switch (dtype) {
    case MSDA_F32: return dispatch_cv<float, float>(cv, f);
    case MSDA_F64: return dispatch_cv<double, double>(cv, f);
    case MSDA_BF16:
      return loc_f32 ? dispatch_cv<bf16_t, float>(cv, f) : dispatch_cv<bf16_t, bf16_t>(cv, f);
    case MSDA_F16:
      return loc_f32 ? dispatch_cv<f16_t, float>(cv, f) : dispatch_cv<f16_t, f16_t>(cv, f);
  }
  return hipErrorInvalidValue;
}

// Launch layout of the backward.
struct BackwardPlan {
  BwdGeom bg;
  int cvr;
  size_t owner_lds;
  int64_t owner_blocks;
  bool bucket;            // try the bucket sort (the kernels re-check on the device)
  size_t bucket_lds;
  int64_t bucket_chunks;  // bucketing workgroups per (b, h)
  int bucket_spt;         // samples per bucketing thread: kBucketSamples, or kBucketSamplesSmall
  int64_t zero_keys;      // bucket counters to clear per (b, h), at most
  int64_t scan_blocks;    // workgroups of msda_bucket_scan_kernel
  bool mfma;              // grad_value on the matrix cores (8 x 8 tiles)
  bool mfma_fallback;     // and the VALU owner kernel after it, for when its counters do not fit
  int fallback_nw;        // that launch's persistent tile slots per (b, h): a small grid, since it
  int64_t fallback_blocks;  // returns at once whenever the matrix-core kernel did the work
  int mfma_nb;            // 16-channel column blocks
  int64_t mfma_blocks;
  size_t mfma_lds;
  int mfma_table;         // entries of its queue's prefix table
  bool small_sort;        // the bucket sort in one launch (msda_bucket_small_kernel)
  int small_sort_keys;    // its LDS counters
  size_t small_sort_lds;
  Plan sample;
};

// The attributes the backward plans with, per device: LDS bytes one workgroup may
// take, and compute units. Read from the runtime on a device's first call and kept
// (a relaxed atomic per field: concurrent first calls store the same values).
struct DeviceInfo {
  std::atomic<int> lds{0}, cus{0};
};
constexpr int kMaxDevices = 64;
DeviceInfo g_devices[kMaxDevices];

void device_info(size_t* lds, int* cus) {
  int dev = 0;
  *lds = 64 * 1024;
  *cus = 256;
  if (hipGetDevice(&dev) != hipSuccess) return;
  if (dev >= 0 && dev < kMaxDevices) {
    const int l = g_devices[dev].lds.load(std::memory_order_relaxed);
    const int c = g_devices[dev].cus.load(std::memory_order_relaxed);
    if (l > 0 && c > 0) {
      *lds = size_t(l);
      *cus = c;
      return;
    }
  }
  int bytes = 0, n = 0;
  if (hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || bytes <= 0)
    bytes = 64 * 1024;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  if (dev >= 0 && dev < kMaxDevices) {
    g_devices[dev].lds.store(bytes, std::memory_order_relaxed);
    g_devices[dev].cus.store(n, std::memory_order_relaxed);
  }
  *lds = size_t(bytes);
  *cus = n;
}

// Kernel paths a test may force (msda_set_path_override), read once per call.
std::atomic<int> g_path_override{0};

// HIP events msda_backward records between its phases on the calling thread
// (msda_set_phase_events): before the sort, after it (and the softmax statistics),
// after grad_value, after grad_sample. Null: none.
constexpr int kPhaseEvents = 4;
thread_local hipEvent_t g_phase_events[kPhaseEvents] = {};
thread_local bool g_phase_events_on = false;

void record_phase(int i, hipStream_t st) {
  if (g_phase_events_on) (void)hipEventRecord(g_phase_events[i], st);
}

size_t owner_lds_bytes(int dtype, int64_t L, int64_t D, int nb, int cap) {
  const size_t es = size_t(elem_size(dtype));
  const size_t rec = dtype == MSDA_F64 ? sizeof(TileRec<double>) : 8;
  size_t at = (sizeof(Level) + sizeof(LevelTiles) + sizeof(int)) * size_t(L) + sizeof(int) * size_t(L + 1);
  at = (at + 15) & ~size_t(15);
  at += 16;
  at += 2 * size_t(nb) * (size_t(D) * es + 16);
  at += rec * size_t(4 * nb);
  at += sizeof(uint32_t) * size_t(nb);
  at += sizeof(int) * size_t(2 * cap + 1);
  return at;
}

int make_backward_plan(int dtype, int64_t B, int64_t S, int64_t H, int64_t D, int64_t Q, int64_t L,
                       int64_t P, int loc_dtype, const void* const* vec_ptrs, int n_vec,
                       const void* grad_attn, size_t lds_limit, int cus, BackwardPlan* plan,
                       bool accumulate = false, int paths = 0, int64_t scratch_bytes = -1) {
  // vec_ptrs: value, grad_output, grad_value (channel vectors), then the locations.
  const int n_chan = std::min(n_vec, 3);
  int rc = make_plan(dtype, B, S, H, D, Q, L, P, true, vec_ptrs, n_chan, &plan->sample, elem_size(loc_dtype));
  if (rc != MSDA_OK) return rc;
  const int es = elem_size(dtype);
  // Channels per register item: the widest power of two that divides D, fits a
  // 16-byte access and keeps grad_out and grad_value aligned to it.
  int cvr = 16 / es;
  while (cvr > 1) {
    bool ok = D % cvr == 0;
    for (int i = 0; i < n_chan && ok; ++i) ok = aligned(vec_ptrs[i], cvr * es);
    if (ok) break;
    cvr >>= 1;
  }
  const int64_t groups = D / cvr;
  if (groups > int64_t(kOwnerThreads) * kOwnerItems)
    return fail(MSDA_ERR_UNSUPPORTED,
                "msda: %lld channels per head exceed the backward's %d register items per workgroup",
                (long long)D, kOwnerThreads * kOwnerItems);
  BwdGeom bg = {};
  bg.groups = int(groups);
  bg.cap = pow2_floor(std::min<int64_t>(kOwnerThreads, int64_t(kOwnerThreads) * kOwnerItems / groups));
  bg.amin = std::min(64, bg.cap);
  bg.nb = pow2_floor(std::min<int64_t>(kOwnerThreads, std::max<int64_t>(1, int64_t(kOwnerThreads) * kOwnerChunks / groups)));
  const size_t budget = lds_limit < 160 * 1024 ? lds_limit : 160 * 1024;
  while (owner_lds_bytes(dtype, L, D, bg.nb, bg.cap) > budget && bg.nb > 1) bg.nb >>= 1;
  if (owner_lds_bytes(dtype, L, D, bg.nb, bg.cap) > budget)
    return fail(MSDA_ERR_UNSUPPORTED, "msda: %lld levels do not fit the backward's LDS budget", (long long)L);
  const int64_t samples_bh = Q * L * P;
  bg.region = samples_bh;
  // The sort's scratch: grad_attention_weights, or the counters region of a workspace.
  const int64_t attn_bytes = scratch_bytes >= 0 ? scratch_bytes : B * samples_bh * H * es;
  const bool attn_ok = (reinterpret_cast<uintptr_t>(grad_attn) & 3) == 0;
  bg.keys_alloc = attn_ok && samples_bh < (int64_t(1) << 32) && B * H > 0 ? attn_bytes / (4 * B * H) : 0;
  // The matrix-core grad_value: float and 16-bit dtypes, D in {16, 32, 48, 64} with
  // 16-byte aligned rows, and its bucket and queue counters (4 per 8 x 8 tile) in the
  // scratch. A level of h x w positions has ceil(h / 8) ceil(w / 8) <= h w / 8 + 1
  // such tiles (the bound of a 1-row level). When that bound does not fit (few queries
  // against a large pyramid, as in a decoder), an estimate for levels of aspect ratio
  // at most 4 decides: ceil(h / 8) ceil(w / 8) <= h w / 64 + (h + w) / 8 + 1 with
  // h + w <= 2.5 sqrt(h w), and sum_l sqrt(h_l w_l) <= sqrt(L S). The kernels then
  // check the real count, and the VALU owner kernel (which takes 8 x 8 tiles when
  // its capacity is at least 64 positions) runs after the matrix-core one and works
  // only if the counters did not fit.
  // A level that takes 4 x 4 tiles (small_tiles) has fewer than kSmallTileTasks / (B H)
  // 8 x 8 tiles, so fewer than four times that many 4 x 4 ones.
  const bool small_tiles = !(paths & MSDA_PATH_TILE8);
  const int64_t small_level_tiles = small_tiles ? 4 * (kSmallTileTasks / std::max<int64_t>(1, B * H) + 1) : 0;
  const int64_t mfma_tiles_bound = L * std::max<int64_t>(S / 8 + 1, small_level_tiles);
  const int64_t mfma_tiles_estimate =
      S / 64 + int64_t(ceil(2.5 * sqrt(double(L) * double(S)) / 8.0)) + 2 * L + (small_tiles ? small_level_tiles : 0);
  const int64_t ls = elem_size(loc_dtype);
  const int64_t per_image = Q * H * std::max(L * P * 2 * ls, D * es);  // 32-bit offsets inside an image
  const bool mfma_sure = 4 * mfma_tiles_bound + kQueueInts <= bg.keys_alloc;
  // The matrix-core kernel's LDS: per wave the staged rows (split for float)
  // and the weight tiles, plus its queue's prefix table of (pair, level) entries: at
  // most kMfmaMaxRegions^2 regions per image, an eighth of the (image, region) pairs per queue.
  const bool mfma_split = dtype == MSDA_F32;
  const int mfma_table = int(std::min<int64_t>(
      kMfmaTable, ((B * kMfmaMaxRegions * kMfmaMaxRegions + kXcds - 1) / kXcds) * L));
  const size_t mfma_lds = mfma_lds_bytes(L, D, mfma_split) + sizeof(int) * size_t(2 * mfma_table + 1);
  const bool mfma_likely = 4 * mfma_tiles_estimate + kQueueInts <= bg.keys_alloc && bg.cap >= 64;
  bool mfma_ok = (dtype == MSDA_BF16 || dtype == MSDA_F16 || dtype == MSDA_F32) && D % 16 == 0 &&
                 D / 16 <= kMfmaMaxNb && (mfma_sure || mfma_likely) &&
                 mfma_lds <= lds_limit &&
                 B * H * mfma_tiles_bound < (int64_t(1) << 31) && per_image < (int64_t(1) << 31) &&
                 !(paths & MSDA_PATH_NO_MFMA);
  for (int i = 0; i < n_chan && mfma_ok; ++i) mfma_ok = aligned(vec_ptrs[i], 16);
  plan->mfma = mfma_ok;
  plan->mfma_fallback = mfma_ok && !mfma_sure;
  bg.sub_log2 = mfma_ok ? kMfmaSubLog2 : 0;
  bg.small_tiles = mfma_ok && small_tiles ? 1 : 0;
  if (mfma_ok) bg.amin = 1 << (2 * kMfmaSubLog2);
  // Tiles per (b, h): every level has at most 3 h w / amin + 1 adaptive tiles.
  const int64_t tiles_bound = mfma_ok ? mfma_tiles_bound : L + 3 * ((L * S + bg.amin - 1) / bg.amin);
  if (tiles_bound >= (int64_t(1) << 29))
    return fail(MSDA_ERR_UNSUPPORTED, "msda: too many backward tiles for S = %lld and L = %lld",
                (long long)S, (long long)L);
  bg.nw = int(std::min<int64_t>(tiles_bound, 2 * ((S + bg.cap - 1) / bg.cap) + L));
  plan->bucket = bg.keys_alloc >= 4 * L;
  if (!plan->bucket) bg.keys_alloc = 0;
  plan->zero_keys = std::min<int64_t>(bg.keys_alloc, 4 * tiles_bound);
  // Bucketing kernels: LDS counters for up to keys_lds buckets (count + base).
  const size_t bucket_head = (((sizeof(Level) + sizeof(LevelTiles)) * size_t(L) + 15) & ~size_t(15)) + 16;
  const int64_t want_keys = std::min<int64_t>(kBucketLdsKeys, plan->zero_keys);
  bg.keys_lds = int(std::max<int64_t>(0, std::min<int64_t>(want_keys, int64_t(budget - std::min(budget, bucket_head)) / 4)));
  plan->bucket_lds = bucket_head + size_t(bg.keys_lds) * 4;
  // Small calls (fewer bucketing workgroups than two per CU) give each thread a few
  // samples, not 32: more workgroups, each a short chain of dependent loads.
  plan->bucket_spt = kBucketSamples;
  if (B * H * ((samples_bh + kBucketThreads * kBucketSamples - 1) / (kBucketThreads * kBucketSamples)) < 2 * cus)
    plan->bucket_spt = kBucketSamplesSmall;
  plan->bucket_chunks = (samples_bh + kBucketThreads * plan->bucket_spt - 1) / (kBucketThreads * plan->bucket_spt);
  plan->owner_blocks = xcd_group_grid(H, int64_t(bg.nw) * B);
  plan->fallback_nw = int(std::max<int64_t>(1, std::min<int64_t>(bg.nw, (2 * int64_t(cus) + B * H - 1) / (B * H))));
  plan->fallback_blocks = xcd_group_grid(H, int64_t(plan->fallback_nw) * B);
  plan->owner_lds = owner_lds_bytes(dtype, L, D, bg.nb, bg.cap);
  plan->mfma_nb = int(D / 16);
  plan->mfma_lds = mfma_lds;
  plan->mfma_table = mfma_table;
  if (mfma_ok) {
    // Persistent workgroups, as many as fit the CUs at once, a multiple of 8.
    const int64_t static_lds = sizeof(int) * (kMfmaWaves + 2 + 3);
    const int64_t per_cu =
        std::max<int64_t>(1, std::min<int64_t>(mfma_blocks_per_cu(int(D / 16), es),
                                               int64_t(160 * 1024) / (int64_t(plan->mfma_lds) + static_lds)));
    const int64_t blocks = std::min<int64_t>(B * H * tiles_bound, int64_t(cus) * per_cu);
    plan->mfma_blocks = (blocks + kXcds - 1) / kXcds * kXcds;
  } else {
    plan->mfma_blocks = 0;
  }
  if (plan->owner_blocks >= 2147483647 || B * H * plan->bucket_chunks >= 2147483647 ||
      B * S >= 2147483647)
    return fail(MSDA_ERR_UNSUPPORTED, "msda: backward grid too large");
  bg.div_lp = make_fastdiv(uint32_t(L * P));
  bg.div_p = make_fastdiv(uint32_t(P));
  // Grouped bucketing: groups of 4 samples, LDS counters for every bucket, and the
  // saved keys (16-bit when every key fits) inside grad_value. Not when grad_value's
  // contents are to be accumulated into: the per-sample passes recompute the keys.
  // The keys of a group are parked as one 8- or 16-byte word, so grad_value must be
  // aligned to it.
  const void* loc_ptr = n_vec > 3 ? vec_ptrs[3] : nullptr;
  const void* gv_ptr = n_vec > 2 ? vec_ptrs[2] : nullptr;
  bg.key_bytes = 4 * tiles_bound < 0xffff ? 2 : 4;
  bg.group4 = !accumulate && (L * P) % 4 == 0 && P % 4 == 0 && plan->bucket &&
              (loc_ptr == nullptr || aligned(loc_ptr, 16)) && (gv_ptr == nullptr || aligned(gv_ptr, 4 * bg.key_bytes));
  if (B * H * samples_bh * bg.key_bytes > B * S * H * D * es) bg.group4 = 0;
  if (!bg.group4) bg.key_bytes = 0;
  // Per-workgroup counts for the grouped passes, where the device finds them room.
  bg.chunks = bg.group4 && !(paths & MSDA_PATH_ATOMIC_SORT) ? int(plan->bucket_chunks) : 0;
  plan->scan_blocks = B * H;
  if (bg.chunks > 0)  // a grid-stride loop over (b, h, bucket) when chunked
    plan->scan_blocks = std::max<int64_t>(plan->scan_blocks, std::min<int64_t>((B * H * plan->zero_keys + 255) / 256, 512));
  if (bg.group4) {
    bg.div_gpq = make_fastdiv(uint32_t(L * P / 4));
    bg.div_gpl = make_fastdiv(uint32_t(P / 4));
  }
  // Small calls: the whole sort in one launch, one workgroup per (b, h), its counters
  // in LDS (as many as the LDS budget holds; the kernel counts in its scratch row
  // otherwise).
  plan->small_sort = plan->bucket && samples_bh <= kSmallSortSamples && (L * P) % 4 == 0 && P % 4 == 0 &&
                     (loc_ptr == nullptr || aligned(loc_ptr, 16)) && !(paths & MSDA_PATH_ATOMIC_SORT);
  plan->small_sort_keys = int(std::max<int64_t>(
      0, std::min<int64_t>(plan->zero_keys, int64_t(budget - std::min(budget, bucket_head + 1024)) / 4)));
  plan->small_sort_lds = bucket_head + size_t(plan->small_sort_keys) * 4;
  if (plan->small_sort) {
    bg.chunks = 0;
    bg.div_gpq = make_fastdiv(uint32_t(L * P / 4));
    bg.div_gpl = make_fastdiv(uint32_t(P / 4));
  }
  plan->bg = bg;
  plan->cvr = cvr;
  return MSDA_OK;
}

template <typename Kernel>
hipError_t allow_lds(Kernel k, size_t bytes) {
  if (bytes <= 64 * 1024) return hipSuccess;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                             int(bytes));
}

template <typename T, typename TL, int CVR, bool SM>
hipError_t launch_owner(const BackwardPlan& plan, const Problem& p, const int* buckets,
                        const uint32_t* entries, int accumulate, int after_mfma, hipStream_t st) {
  auto k = msda_grad_value_kernel<T, TL, CVR, SM>;
  const hipError_t e = allow_lds(k, plan.owner_lds);
  if (e != hipSuccess) return e;
  BwdGeom bg = plan.bg;
  int64_t blocks = plan.owner_blocks;
  if (after_mfma) {
    bg.nw = plan.fallback_nw;
    blocks = plan.fallback_blocks;
  }
  hipLaunchKernelGGL(k, dim3(unsigned(blocks)), dim3(kOwnerThreads), plan.owner_lds, st, p, bg, buckets, entries,
                     accumulate, after_mfma);
  return hipGetLastError();
}

template <typename T, typename TL, bool SM>
hipError_t launch_owner_cvr(const BackwardPlan& plan, const Problem& p, const int* buckets,
                            const uint32_t* entries, int accumulate, int after_mfma, hipStream_t st) {
  constexpr int kMaxCv = 16 / Elem<T>::size;
  switch (plan.cvr) {
    case 1: return launch_owner<T, TL, 1, SM>(plan, p, buckets, entries, accumulate, after_mfma, st);
    case 2: return launch_owner<T, TL, 2, SM>(plan, p, buckets, entries, accumulate, after_mfma, st);
    case 4:
      if constexpr (kMaxCv >= 4)
        return launch_owner<T, TL, 4, SM>(plan, p, buckets, entries, accumulate, after_mfma, st);
      break;
    case 8:
      if constexpr (kMaxCv >= 8)
        return launch_owner<T, TL, 8, SM>(plan, p, buckets, entries, accumulate, after_mfma, st);
      break;
  }
  return hipErrorInvalidValue;
}

template <typename T, typename TL, bool SM>
hipError_t launch_owner_mfma(const BackwardPlan& plan, const Problem& p, const int* buckets,
                             const uint32_t* entries, int accumulate, hipStream_t st) {
  if constexpr (std::is_same_v<T, bf16_t> || std::is_same_v<T, f16_t> || std::is_same_v<T, float>) {
    auto go = [&](auto k) -> hipError_t {
      const hipError_t e = allow_lds(k, plan.mfma_lds);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(k, dim3(unsigned(plan.mfma_blocks)), dim3(kWave * kMfmaWaves), plan.mfma_lds, st, p,
                         plan.bg, const_cast<int*>(buckets), entries, accumulate, plan.mfma_table);
      return hipGetLastError();
    };
    switch (plan.mfma_nb) {
      case 1: return go(msda_grad_value_mfma_kernel<T, TL, 1, SM>);
      case 2: return go(msda_grad_value_mfma_kernel<T, TL, 2, SM>);
      case 3: return go(msda_grad_value_mfma_kernel<T, TL, 3, SM>);
      case 4: return go(msda_grad_value_mfma_kernel<T, TL, 4, SM>);
    }
  }
  return hipErrorInvalidValue;
}

// The count, scan and place passes with SPT samples per bucketing thread.
template <typename TL, int SPT>
hipError_t launch_bucket_passes(const BackwardPlan& plan, const Problem& p, int* buckets, uint32_t* entries,
                                hipStream_t st) {
  const dim3 grid(unsigned(xcd_group_grid(p.H, int64_t(p.B) * plan.bucket_chunks))), block(kBucketThreads);
  const size_t scan_lds = p.L > kMaxOrderedLevels ? (sizeof(Level) + sizeof(LevelTiles)) * size_t(p.L) : 0;
  if (plan.bg.group4) {
    auto run = [&](auto count, auto place) -> hipError_t {
      hipError_t e = allow_lds(count, plan.bucket_lds);
      if (e == hipSuccess) e = allow_lds(place, plan.bucket_lds);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(count, grid, block, plan.bucket_lds, st, p, plan.bg, buckets, entries,
                         int(plan.bucket_chunks));
      hipLaunchKernelGGL(msda_bucket_scan_kernel, dim3(unsigned(plan.scan_blocks)), dim3(256), scan_lds, st, p,
                         plan.bg, buckets, int(plan.bucket_chunks));
      hipLaunchKernelGGL(place, grid, block, plan.bucket_lds, st, p, plan.bg, buckets, entries,
                         int(plan.bucket_chunks));
      return hipGetLastError();
    };
    return plan.bg.key_bytes == 2
               ? run(msda_bucket4_kernel<TL, false, 2, SPT>, msda_bucket4_kernel<TL, true, 2, SPT>)
               : run(msda_bucket4_kernel<TL, false, 4, SPT>, msda_bucket4_kernel<TL, true, 4, SPT>);
  }
  auto count = msda_bucket_kernel<TL, false, SPT>;
  auto place = msda_bucket_kernel<TL, true, SPT>;
  hipError_t e = allow_lds(count, plan.bucket_lds);
  if (e == hipSuccess) e = allow_lds(place, plan.bucket_lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(count, grid, block, plan.bucket_lds, st, p, plan.bg, buckets, entries,
                     int(plan.bucket_chunks));
  hipLaunchKernelGGL(msda_bucket_scan_kernel, dim3(unsigned(plan.scan_blocks)), dim3(256), scan_lds, st, p,
                     plan.bg, buckets, int(plan.bucket_chunks));
  hipLaunchKernelGGL(place, grid, block, plan.bucket_lds, st, p, plan.bg, buckets, entries,
                     int(plan.bucket_chunks));
  return hipGetLastError();
}

// The bucket sort: clear the counters, count, scan, place.
template <typename TL>
hipError_t launch_buckets(const BackwardPlan& plan, const Problem& p, int* buckets, uint32_t* entries,
                          hipStream_t st) {
  if (plan.small_sort) {
    auto k = msda_bucket_small_kernel<TL>;
    const hipError_t e = allow_lds(k, plan.small_sort_lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k, dim3(unsigned(int64_t(p.B) * p.H)), dim3(kSmallSortThreads), plan.small_sort_lds, st, p,
                       plan.bg, buckets, entries, plan.small_sort_keys);
    return hipGetLastError();
  }
  {
    const int64_t n = int64_t(p.B) * p.H * plan.zero_keys;
    const unsigned blocks = unsigned(std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, 1024)));
    const size_t lds = p.L > kMaxOrderedLevels ? (sizeof(Level) + sizeof(LevelTiles)) * size_t(p.L) : 0;
    hipLaunchKernelGGL(msda_bucket_clear_kernel, dim3(blocks), dim3(256), lds, st, p, plan.bg, buckets);
  }
  if (plan.bucket_spt == kBucketSamplesSmall)
    return launch_bucket_passes<TL, kBucketSamplesSmall>(plan, p, buckets, entries, st);
  return launch_bucket_passes<TL, kBucketSamples>(plan, p, buckets, entries, st);
}


int check_call(int value_dtype, int index_dtype, int loc_dtype, int64_t B, int64_t S, int64_t H,
               int64_t D, int64_t Q, int64_t L, int64_t P, int flags, int allowed_flags) {
  if (elem_size(value_dtype) == 0)
    return fail(MSDA_ERR_INVALID, "msda: unknown value dtype code %d", value_dtype);
  if (index_dtype != MSDA_I64 && index_dtype != MSDA_I32)
    return fail(MSDA_ERR_INVALID, "msda: unknown index dtype code %d", index_dtype);
  if (elem_size(loc_dtype) == 0)
    return fail(MSDA_ERR_INVALID, "msda: unknown location dtype code %d", loc_dtype);
  const bool loc_ok = loc_dtype == value_dtype || (loc_dtype == MSDA_F32 && value_dtype != MSDA_F64);
  if (!loc_ok)
    return fail(MSDA_ERR_UNSUPPORTED,
                "msda: %s locations with %s values; locations must be float32 or the value dtype",
                dtype_name(loc_dtype), dtype_name(value_dtype));
  if (flags & ~allowed_flags) return fail(MSDA_ERR_INVALID, "msda: unknown flag bits 0x%x", flags);
  if (B < 0 || S < 0 || H < 0 || D < 0 || Q < 0 || L < 0 || P < 0)
    return fail(MSDA_ERR_INVALID,
                "msda: negative size (B=%lld S=%lld H=%lld D=%lld Q=%lld L=%lld P=%lld)",
                (long long)B, (long long)S, (long long)H, (long long)D, (long long)Q,
                (long long)L, (long long)P);
  const int64_t kInt32 = 2147483647;
  if (B >= kInt32 || S >= kInt32 || H >= kInt32 || D >= kInt32 || Q >= kInt32 || L >= kInt32 ||
      P >= kInt32)
    return fail(MSDA_ERR_UNSUPPORTED, "msda: a size exceeds the int32 range");
  return MSDA_OK;
}

int zero_fill(void* ptr, int64_t bytes, hipStream_t stream, const char* who) {
  const int64_t chunks = bytes / 16 + 1;
  const int64_t want = (chunks + 255) / 256;
  const unsigned blocks = unsigned(want < 4096 ? want : 4096);
  hipLaunchKernelGGL(zero_fill_kernel, dim3(blocks), dim3(256), 0, stream, static_cast<char*>(ptr),
                     bytes);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return fail(MSDA_ERR_HIP, "%s: zero-fill launch failed: %s", who, hipGetErrorString(err));
  return MSDA_OK;
}

// The widest piece (16, 8, 4, 2 or 1 bytes) that divides a unit's bytes and the
// alignment of ptr, for the LDS copy of a wave's locations or weights.
int copy_piece(int64_t unit_bytes, const void* ptr) {
  for (int pc = 16; pc > 1; pc >>= 1)
    if (unit_bytes % pc == 0 && aligned(ptr, pc)) return pc;
  return 1;
}

Problem make_problem(const void* value, const void* shapes, const void* starts, int index_dtype,
                     const void* loc, const void* attn, int64_t B, int64_t S, int64_t H, int64_t D,
                     int64_t Q, int64_t L, int64_t P, const Plan& plan) {
  Problem p = {};
  p.value = static_cast<const char*>(value);
  p.shapes = shapes;
  p.starts = starts;
  p.loc = static_cast<const char*>(loc);
  p.attn = static_cast<const char*>(attn);
  p.index_i32 = index_dtype == MSDA_I32;
  p.B = int(B);
  p.S = int(S);
  p.H = int(H);
  p.D = int(D);
  p.Q = int(Q);
  p.L = int(L);
  p.P = int(P);
  p.lh_log2 = plan.lh_log2;
  p.units_per_block = plan.units_per_block;
  p.blocks_per_batch = plan.blocks_per_batch;
  p.num_blocks = int(plan.num_blocks);
  return p;
}

// The backward's workspace: one uint32 sample index per sample, then the sort's
// counters, count rows and softmax statistics in the rest (at least as many bytes as
// grad_attention_weights, the capacity they have there). msda_backward_workspace_size
// adds room for the bucket and queue counters of the largest tile count the host
// cannot rule out, so that the matrix-core owners never need the VALU kernel's
// standby launch (4 x 4 tiles on small levels included; at most a few MB), and, for
// the softmax method, a region of its own for the per-unit softmax statistics, which
// grad_sample then writes on its side stream.
struct WorkspaceLayout {
  int64_t counters_off, counters_bytes, stats_off, base, total;
};

WorkspaceLayout workspace_layout(int dtype, int64_t B, int64_t S, int64_t H, int64_t Q, int64_t L, int64_t P,
                                 bool softmax) {
  auto align = [](int64_t v) { return (v + 255) / 256 * 256; };
  const int64_t samples = B * Q * H * L * P;
  const int64_t small_level_tiles = 4 * (kSmallTileTasks / std::max<int64_t>(1, B * H) + 1);
  const int64_t tiles_bound = L * std::max<int64_t>(S / 8 + 1, small_level_tiles);
  const int64_t counters = B * H * (4 * tiles_bound + kQueueInts) * 4;
  const int64_t stat_bytes = dtype == MSDA_F64 ? 8 : 4;  // SoftStat of the accumulation type
  WorkspaceLayout w;
  w.counters_off = align(samples * 4);
  w.counters_bytes = align(std::max(samples * elem_size(dtype), counters));
  w.base = w.counters_off + align(samples * elem_size(dtype));
  w.stats_off = w.counters_off + w.counters_bytes;
  w.total = w.stats_off + (softmax ? align(B * Q * H * stat_bytes) : 0);
  return w;
}

// Calls of fewer samples keep one stream. The overlap saves GPU time in proportion
// to the samples (MI355X: 2.6 us more at 129 K samples, 5 us less at 1 M, 10-37 us
// less at 4.6-8.3 M), but the fork and join cost the calling thread about 45 us
// (two hipStreamWaitEvent calls of 12-16 us each and a launch on a second queue,
// against 14 us for the whole one-stream call). Where the backward's GPU time is
// not well above the host time of a training step, that delay is the step's.
constexpr int64_t kSideStreamSamples = int64_t(1) << 21;

struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};

SideStream* side_stream() {
  thread_local SideStream streams[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  SideStream& s = streams[dev];
  if (s.stream == nullptr) {
    if (hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking) != hipSuccess) return nullptr;
    if (hipEventCreateWithFlags(&s.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&s.join, hipEventDisableTiming) != hipSuccess) {
      s.stream = nullptr;
      return nullptr;
    }
  }
  return &s;
}

template <typename T, typename TL, int CV>
hipError_t launch_grad_sample(const BackwardPlan& plan, const Problem& p, bool softmax, hipStream_t st) {
  const dim3 grid(unsigned(plan.sample.num_blocks)), block(unsigned(kWave * plan.sample.waves));
  if (softmax)
    hipLaunchKernelGGL((msda_grad_sample_kernel<T, TL, CV, true>), grid, block, plan.sample.lds, st, p);
  else
    hipLaunchKernelGGL((msda_grad_sample_kernel<T, TL, CV, false>), grid, block, plan.sample.lds, st, p);
  return hipGetLastError();
}

}  // namespace

// The scratch of msda_backward_no_alloc: the workspace msda_backward_workspace takes,
// as a device array the code object brings (no allocation at call time). Each device
// holds its own copy from the module's load on that device until the process ends.
// 64 MiB holds the workspace of every batch of 2^23 samples or fewer in any dtype up
// to 4 bytes (B = 4, Q = 21,504, H = 8, L = 3, P = 4: 66,060,288 bytes in float32).
constexpr int64_t kScratchBytes = int64_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

// `scratch` in host code is the host-side shadow of the device array, not a device
// address: the device address comes from hipGetSymbolAddress, once per device with
// that device current, and is kept.
struct ScratchSlot {
  std::atomic<void*> addr{nullptr};
};
ScratchSlot g_scratch[kMaxDevices];

int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(MSDA_ERR_HIP, "msda_backward_no_alloc: no current device: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MSDA_ERR_INVALID, "msda_backward_no_alloc: device %d beyond the %d the library tracks", dev,
                kMaxDevices);
  void* addr = g_scratch[dev].addr.load(std::memory_order_acquire);
  if (addr == nullptr) {
    // Concurrent first calls on one device look up the same address.
    e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || addr == nullptr)
      return fail(MSDA_ERR_HIP, "msda_backward_no_alloc: hipGetSymbolAddress(scratch) failed: %s",
                  hipGetErrorString(e));
    g_scratch[dev].addr.store(addr, std::memory_order_release);
  }
  *out = addr;
  return MSDA_OK;
}

}  // namespace

extern "C" {

const char* msda_last_error(void) { return g_last_error; }

int msda_abi_version(void) { return MSDA_ABI_VERSION; }

int msda_set_phase_events(void* const* events, int count) {
  g_last_error[0] = '\0';
  if (count == 0) {
    g_phase_events_on = false;
    return MSDA_OK;
  }
  if (count != kPhaseEvents || events == nullptr)
    return fail(MSDA_ERR_INVALID, "msda_set_phase_events: give %d events, or 0 to stop", kPhaseEvents);
  for (int i = 0; i < kPhaseEvents; ++i) {
    if (events[i] == nullptr) return fail(MSDA_ERR_INVALID, "msda_set_phase_events: null event %d", i);
    g_phase_events[i] = static_cast<hipEvent_t>(events[i]);
  }
  g_phase_events_on = true;
  return MSDA_OK;
}

int msda_set_path_override(int paths) {
  return g_path_override.exchange(paths & (MSDA_PATH_NO_MFMA | MSDA_PATH_ATOMIC_SORT | MSDA_PATH_TILE8),
                                  std::memory_order_relaxed);
}

int msda_launch_geometry(int value_dtype, int64_t batch, int64_t spatial, int64_t heads,
                         int64_t channels, int64_t queries, int64_t levels, int64_t points,
                         int backward, int* channels_per_lane, int* lanes_per_unit,
                         int* waves_per_block, int64_t* num_blocks) {
  if (elem_size(value_dtype) == 0)
    return fail(MSDA_ERR_INVALID, "msda: unknown value dtype code %d", value_dtype);
  if (backward) {
    BackwardPlan bp;
    const int rc = make_backward_plan(value_dtype, batch, spatial, heads, channels, queries,
                                      levels, points, value_dtype, nullptr, 0, nullptr, 160 * 1024, 256,
                                      &bp);
    if (rc != MSDA_OK) return rc;
    // The grad_value kernel's layout: channels per register item, positions per
    // tile at most, waves per workgroup and workgroups.
    if (channels_per_lane) *channels_per_lane = bp.cvr;
    if (lanes_per_unit) *lanes_per_unit = bp.bg.cap;
    if (waves_per_block) *waves_per_block = kOwnerThreads / kWave;
    if (num_blocks) *num_blocks = bp.owner_blocks;
    return MSDA_OK;
  }
  Plan plan;
  const int rc = make_plan(value_dtype, batch, spatial, heads, channels, queries, levels, points,
                           false, nullptr, 0, &plan, elem_size(value_dtype));
  if (rc != MSDA_OK) return rc;
  if (channels_per_lane) *channels_per_lane = plan.cv;
  if (lanes_per_unit) *lanes_per_unit = 1 << plan.lh_log2;
  if (waves_per_block) *waves_per_block = plan.waves;
  if (num_blocks) *num_blocks = plan.num_blocks;
  return MSDA_OK;
}

int msda_forward(const void* value, int value_dtype, const void* spatial_shapes,
                 const void* level_start_index, int index_dtype, const void* sampling_locations,
                 int loc_dtype, const void* attention_weights, void* output, int64_t batch,
                 int64_t spatial, int64_t heads, int64_t channels, int64_t queries,
                 int64_t levels, int64_t points, int flags, void* stream) {
  g_last_error[0] = '\0';
  int rc = check_call(value_dtype, index_dtype, loc_dtype, batch, spatial, heads, channels,
                      queries, levels, points, flags, MSDA_SOFTMAX);
  if (rc != MSDA_OK) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t out_bytes = batch * queries * heads * channels * elem_size(value_dtype);
  if (out_bytes == 0) return MSDA_OK;
  if (!output) return fail(MSDA_ERR_INVALID, "msda_forward: null output");
  (void)hipGetLastError();
  // No sample, or nothing to sample from: the output is all zeros.
  if (levels * points == 0 || spatial == 0) return zero_fill(output, out_bytes, st, "msda_forward");
  if (!value || !spatial_shapes || !level_start_index || !sampling_locations || !attention_weights)
    return fail(MSDA_ERR_INVALID, "msda_forward: null input tensor pointer");
  const void* vec[] = {value, output};
  Plan plan;
  rc = make_plan(value_dtype, batch, spatial, heads, channels, queries, levels, points, false,
                 vec, 2, &plan, elem_size(loc_dtype));
  if (rc != MSDA_OK) return rc;
  Problem p = make_problem(value, spatial_shapes, level_start_index, index_dtype,
                           sampling_locations, attention_weights, batch, spatial, heads,
                           channels, queries, levels, points, plan);
  p.loc_piece = copy_piece(levels * points * 2 * elem_size(loc_dtype), sampling_locations);
  p.attn_piece = copy_piece(levels * points * elem_size(value_dtype), attention_weights);
  p.out = static_cast<char*>(output);
  const bool softmax = flags & MSDA_SOFTMAX;
  const hipError_t err = dispatch(
      value_dtype, loc_dtype == MSDA_F32 && value_dtype != MSDA_F32, plan.cv,
      [&]<typename T, typename TL, int CV>() {
        const dim3 grid(unsigned(plan.num_blocks)), block(unsigned(kWave * plan.waves));
        if (softmax)
          hipLaunchKernelGGL((msda_forward_kernel<T, TL, CV, true>), grid, block, plan.lds, st, p);
        else
          hipLaunchKernelGGL((msda_forward_kernel<T, TL, CV, false>), grid, block, plan.lds, st, p);
        return hipGetLastError();
      });
  if (err != hipSuccess)
    return fail(MSDA_ERR_HIP, "msda_forward: launch failed: %s", hipGetErrorString(err));
  return MSDA_OK;
}

// msda_backward (workspace null) and msda_backward_workspace.
static int backward_call(const void* value, int value_dtype, const void* spatial_shapes,
                         const void* level_start_index, int index_dtype, const void* sampling_locations,
                         int loc_dtype, const void* attention_weights, const void* grad_output,
                         void* grad_value, void* grad_sampling_locations, void* grad_attention_weights,
                         int64_t batch, int64_t spatial, int64_t heads, int64_t channels,
                         int64_t queries, int64_t levels, int64_t points, int flags, void* workspace,
                         int64_t workspace_bytes, bool fork, void* stream) {
  g_last_error[0] = '\0';
  int rc = check_call(value_dtype, index_dtype, loc_dtype, batch, spatial, heads, channels,
                      queries, levels, points, flags,
                      MSDA_SOFTMAX | MSDA_ACCUMULATE_GRAD_VALUE | MSDA_GRAD_VALUE_ATOMIC);
  if (rc != MSDA_OK) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int es = elem_size(value_dtype);
  const int64_t value_bytes = batch * spatial * heads * channels * es;
  const int64_t sample_count = batch * queries * heads * levels * points;
  if (value_bytes > 0 && !grad_value)
    return fail(MSDA_ERR_INVALID, "msda_backward: null grad_value");
  if (sample_count > 0 && (!grad_sampling_locations || !grad_attention_weights))
    return fail(MSDA_ERR_INVALID, "msda_backward: null location or weight gradient");
  const bool accumulate = flags & MSDA_ACCUMULATE_GRAD_VALUE;
  const bool atomic_gv = flags & MSDA_GRAD_VALUE_ATOMIC;
  (void)hipGetLastError();
  if (sample_count == 0 || channels == 0 || spatial == 0) {
    // Nothing to sample: grad_value keeps its contents (accumulate) or becomes zero,
    // and every location and weight gradient is zero.
    if (value_bytes > 0 && !accumulate) {
      rc = zero_fill(grad_value, value_bytes, st, "msda_backward");
      if (rc != MSDA_OK) return rc;
    }
    if (sample_count == 0) return MSDA_OK;
    rc = zero_fill(grad_sampling_locations, sample_count * 2 * elem_size(loc_dtype), st,
                   "msda_backward");
    if (rc != MSDA_OK) return rc;
    return zero_fill(grad_attention_weights, sample_count * es, st, "msda_backward");
  }
  if (!value || !spatial_shapes || !level_start_index || !sampling_locations ||
      !attention_weights || !grad_output)
    return fail(MSDA_ERR_INVALID, "msda_backward: null input tensor pointer");
  if (reinterpret_cast<uintptr_t>(grad_sampling_locations) % 4 != 0)
    return fail(MSDA_ERR_INVALID, "msda_backward: grad_sampling_locations must be 4-byte aligned");
  const void* vec[] = {value, grad_output, grad_value, sampling_locations};
  // The sort's scratch: the caller's workspace when it is large enough (then
  // grad_sample may run beside the sort), else grad_attention_weights and
  // grad_sampling_locations (then grad_sample runs last).
  const bool softmax = flags & MSDA_SOFTMAX;
  const WorkspaceLayout wl = workspace_layout(value_dtype, batch, spatial, heads, queries, levels, points, softmax);
  const bool use_ws = workspace != nullptr && workspace_bytes >= wl.base && aligned(workspace, 256);
  // A workspace of the full size gives the softmax statistics a region of their own.
  const bool ws_stats = use_ws && softmax && workspace_bytes >= wl.total;
  void* counters = use_ws ? static_cast<char*>(workspace) + wl.counters_off : grad_attention_weights;
  BackwardPlan plan;
  size_t lds_limit;
  int cus;
  device_info(&lds_limit, &cus);
  rc = make_backward_plan(value_dtype, batch, spatial, heads, channels, queries, levels, points,
                          loc_dtype, vec, 4, counters, lds_limit, cus, &plan, accumulate,
                          g_path_override.load(std::memory_order_relaxed),
                          !use_ws ? -1 : ws_stats ? wl.counters_bytes : workspace_bytes - wl.counters_off);
  if (rc != MSDA_OK) return rc;
  Problem p = make_problem(value, spatial_shapes, level_start_index, index_dtype,
                           sampling_locations, attention_weights, batch, spatial, heads,
                           channels, queries, levels, points, plan.sample);
  p.loc_piece = copy_piece(levels * points * 2 * elem_size(loc_dtype), sampling_locations);
  p.attn_piece = copy_piece(levels * points * elem_size(value_dtype), attention_weights);
  p.grad_out = static_cast<const char*>(grad_output);
  p.grad_value = static_cast<char*>(grad_value);
  p.grad_loc = static_cast<char*>(grad_sampling_locations);
  p.grad_attn = static_cast<char*>(grad_attention_weights);
  p.atomic_gv = atomic_gv ? 1 : 0;
  // The matrix-core owners take overlapping levels when nothing falls back to the
  // VALU owner kernel (which stores, and stands aside on overlap).
  p.sort_overlap = plan.bucket && plan.mfma && !plan.mfma_fallback && !atomic_gv ? 1 : 0;
  p.zero_gv = accumulate ? 0 : 1;
  p.es = es;
  if (atomic_gv && !accumulate) {  // the atomic scatter adds into zeros
    rc = zero_fill(grad_value, value_bytes, st, "msda_backward");
    if (rc != MSDA_OK) return rc;
  }
  // Scratch of the bucket sort: counters in grad_attention_weights, sample indices in
  // grad_sampling_locations, which msda_grad_sample_kernel overwrites last; or the
  // workspace.
  int* buckets = static_cast<int*>(counters);
  uint32_t* entries = use_ws ? static_cast<uint32_t*>(workspace) : static_cast<uint32_t*>(grad_sampling_locations);
  // grad_sample beside the sort: it needs neither the sort nor grad_value, and with
  // the scratch in the workspace it writes nothing the sort uses. Only where it adds
  // nothing into grad_value (the matrix-core owners take every level, overlapping ones
  // included); it joins the caller's stream before the grad_value kernel.
  SideStream* side = nullptr;
  if (fork && use_ws && p.sort_overlap && sample_count >= kSideStreamSamples && !g_phase_events_on) {
    side = side_stream();
    if (side == nullptr) return fail(MSDA_ERR_HIP, "msda_backward_workspace: no side stream: %s", hipGetErrorString(hipGetLastError()));
    // grad_sample, which forms each unit's softmax anyway, leaves the statistics for
    // the grad_value kernel in the workspace: no statistics pass after the sort.
    if (ws_stats) p.stats = static_cast<char*>(workspace) + wl.stats_off;
  }
  const hipError_t err = dispatch(
      value_dtype, loc_dtype == MSDA_F32 && value_dtype != MSDA_F32, plan.sample.cv,
      [&]<typename T, typename TL, int CV>() {
        hipError_t e = hipSuccess;
        if (side) {  // fork: grad_sample on the side stream, after the caller's prior work
          e = hipEventRecord(side->fork, st);
          if (e == hipSuccess) e = hipStreamWaitEvent(side->stream, side->fork, 0);
          if (e == hipSuccess) e = launch_grad_sample<T, TL, CV>(plan, p, softmax, side->stream);
          if (e == hipSuccess) e = hipEventRecord(side->join, side->stream);
          if (e != hipSuccess) return e;
        }
        record_phase(0, st);
        // The atomic scatter needs neither the sort nor the owners.
        if (plan.bucket && !atomic_gv) {
          e = launch_buckets<TL>(plan, p, buckets, entries, st);
          if (e != hipSuccess) return e;
          if (softmax && !p.stats) {  // per-unit softmax statistics, where the scratch has room
            const int64_t units = int64_t(p.B) * p.Q * p.H;
            const unsigned blocks = unsigned(std::max<int64_t>(1, std::min<int64_t>((units + 255) / 256, 2048)));
            const size_t lds = p.L > kMaxOrderedLevels ? (sizeof(Level) + sizeof(LevelTiles)) * size_t(p.L) : 0;
            hipLaunchKernelGGL((msda_softmax_stats_kernel<T>), dim3(blocks), dim3(256), lds, st, p, plan.bg,
                               buckets);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
          }
        }
        record_phase(1, st);
        if (!accumulate && !plan.mfma && !atomic_gv) {  // the matrix-core kernel zeroes the gaps itself
          const int64_t n = int64_t(p.B) * p.S;
          hipLaunchKernelGGL((msda_gap_zero_kernel<T>), dim3(unsigned((n + 255) / 256)), dim3(256),
                             sizeof(Level) * size_t(p.L), st, p);
          e = hipGetLastError();
          if (e != hipSuccess) return e;
        }
        // The join: before the grad_value kernel when it reads the softmax statistics
        // grad_sample leaves; otherwise after it, so that grad_sample's tail overlaps it.
        if (side && p.stats) {
          e = hipStreamWaitEvent(st, side->join, 0);
          if (e != hipSuccess) return e;
        }
        if (plan.mfma && !atomic_gv)
          e = softmax ? launch_owner_mfma<T, TL, true>(plan, p, buckets, entries, int(accumulate), st)
                      : launch_owner_mfma<T, TL, false>(plan, p, buckets, entries, int(accumulate), st);
        if (e == hipSuccess && side && !p.stats) e = hipStreamWaitEvent(st, side->join, 0);
        if (e == hipSuccess && !atomic_gv && (!plan.mfma || plan.mfma_fallback)) {
          const int after_mfma = plan.mfma ? 1 : 0;
          e = softmax ? launch_owner_cvr<T, TL, true>(plan, p, buckets, entries, int(accumulate), after_mfma, st)
                      : launch_owner_cvr<T, TL, false>(plan, p, buckets, entries, int(accumulate), after_mfma, st);
        }
        if (e != hipSuccess || side) return e;
        record_phase(2, st);
        e = launch_grad_sample<T, TL, CV>(plan, p, softmax, st);
        record_phase(3, st);
        return e;
      });
  if (err != hipSuccess)
    return fail(MSDA_ERR_HIP, "msda_backward: launch failed: %s", hipGetErrorString(err));
  return MSDA_OK;
}


int msda_backward(const void* value, int value_dtype, const void* spatial_shapes,
                  const void* level_start_index, int index_dtype, const void* sampling_locations,
                  int loc_dtype, const void* attention_weights, const void* grad_output,
                  void* grad_value, void* grad_sampling_locations, void* grad_attention_weights,
                  int64_t batch, int64_t spatial, int64_t heads, int64_t channels,
                  int64_t queries, int64_t levels, int64_t points, int flags, void* stream) {
  return backward_call(value, value_dtype, spatial_shapes, level_start_index, index_dtype, sampling_locations,
                       loc_dtype, attention_weights, grad_output, grad_value, grad_sampling_locations,
                       grad_attention_weights, batch, spatial, heads, channels, queries, levels, points, flags,
                       nullptr, 0, false, stream);
}

int msda_backward_workspace_size(int value_dtype, int64_t batch, int64_t spatial, int64_t heads,
                                 int64_t channels, int64_t queries, int64_t levels, int64_t points, int flags,
                                 int64_t* bytes) {
  g_last_error[0] = '\0';
  if (!bytes) return fail(MSDA_ERR_INVALID, "msda_backward_workspace_size: null result pointer");
  *bytes = 0;
  if (elem_size(value_dtype) == 0)
    return fail(MSDA_ERR_INVALID, "msda: unknown value dtype code %d", value_dtype);
  if (batch < 0 || spatial < 0 || heads < 0 || channels < 0 || queries < 0 || levels < 0 || points < 0)
    return fail(MSDA_ERR_INVALID, "msda: negative size");
  (void)channels;
  *bytes = workspace_layout(value_dtype, batch, spatial, heads, queries, levels, points, flags & MSDA_SOFTMAX).total;
  return MSDA_OK;
}

int msda_backward_workspace(const void* value, int value_dtype, const void* spatial_shapes,
                            const void* level_start_index, int index_dtype, const void* sampling_locations,
                            int loc_dtype, const void* attention_weights, const void* grad_output,
                            void* grad_value, void* grad_sampling_locations, void* grad_attention_weights,
                            int64_t batch, int64_t spatial, int64_t heads, int64_t channels,
                            int64_t queries, int64_t levels, int64_t points, int flags, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  if (workspace_bytes < 0) return fail(MSDA_ERR_INVALID, "msda_backward_workspace: negative workspace size");
  return backward_call(value, value_dtype, spatial_shapes, level_start_index, index_dtype, sampling_locations,
                       loc_dtype, attention_weights, grad_output, grad_value, grad_sampling_locations,
                       grad_attention_weights, batch, spatial, heads, channels, queries, levels, points, flags,
                       workspace, workspace_bytes, true, stream);
}

int msda_backward_no_alloc(const void* value, int value_dtype, const void* spatial_shapes,
                           const void* level_start_index, int index_dtype, const void* sampling_locations,
                           int loc_dtype, const void* attention_weights, const void* grad_output,
                           void* grad_value, void* grad_sampling_locations, void* grad_attention_weights,
                           int64_t batch, int64_t spatial, int64_t heads, int64_t channels,
                           int64_t queries, int64_t levels, int64_t points, int flags, void* stream) {
  g_last_error[0] = '\0';
  int rc = check_call(value_dtype, index_dtype, loc_dtype, batch, spatial, heads, channels,
                      queries, levels, points, flags,
                      MSDA_SOFTMAX | MSDA_ACCUMULATE_GRAD_VALUE | MSDA_GRAD_VALUE_ATOMIC);
  if (rc != MSDA_OK) return rc;
  const int64_t need = workspace_layout(value_dtype, batch, spatial, heads, queries, levels, points, false).base;
  if (need > kScratchBytes)
    return fail(MSDA_ERR_INVALID,
                "msda_backward_no_alloc: these sizes need %lld bytes of scratch, the static scratch holds %lld "
                "(use msda_backward_workspace)",
                static_cast<long long>(need), static_cast<long long>(kScratchBytes));
  void* ws = nullptr;
  rc = scratch_address(&ws);
  if (rc != MSDA_OK) return rc;
  return backward_call(value, value_dtype, spatial_shapes, level_start_index, index_dtype, sampling_locations,
                       loc_dtype, attention_weights, grad_output, grad_value, grad_sampling_locations,
                       grad_attention_weights, batch, spatial, heads, channels, queries, levels, points, flags,
                       ws, kScratchBytes, false, stream);
}

}  // extern "C"
