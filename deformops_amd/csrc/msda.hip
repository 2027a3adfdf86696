// Multi-scale deformable attention (MSDA) for AMD Instinct MI355X (gfx950):
// forward and zero-buffer backward behind the C ABI of include/deformops_amd.h.
//
// Work decomposition. A "unit" is one (batch, query, head): it owns the D channels
// of one output vector and L * P samples. A unit is served by LH = 2^k lanes of a
// wave64, each lane holding CV consecutive channels (CV * element size <= 16 bytes,
// so one corner fetch is one global_load_dwordx4 for bf16/f16 D = 32). A wave
// therefore serves UW = 64 / LH units; a workgroup is 1-4 waves. Workgroups are
// renumbered so that consecutive units land on the same XCD (gfx950 deals
// workgroups to its 8 XCDs round-robin, and each XCD has its own L2): queries that
// are neighbours in the flattened pyramid sample neighbouring pixels, so this keeps
// their corner gathers and grad_value atomics inside one L2.
//
// Each kernel runs in phases:
//   1. Every lane of a unit takes samples s = t, t + LH, ... (t = lane in unit),
//      reads its location and weight, and stages the sample's four corner byte
//      offsets and four (bilinear * attention) weights in LDS. The softmax over the
//      L * P weights of a unit is a cross-lane max / sum inside the unit's lanes.
//   2. The unit's lanes walk all L * P samples: one broadcast LDS read of the
//      staged sample, four vector corner loads, fp32 (fp64 for double) FMAs.
//      The backward also forms the four per-corner dot products
//      G_c = sum_d grad_out[d] * value_c[d], reduces them across the unit's lanes,
//      and scatters grad_out * weight into grad_value with global atomics in the
//      value dtype (global_atomic_pk_add_bf16 / pk_add_f16 / add_f32 / add_f64).
//   3. (backward) The lane that staged sample s turns its G_c into the location
//      and weight gradients:
//        dL/dw   = sum_c bilinear_c * G_c
//        dL/dx   = a * W * ((1 - dy) (G01 - G00) + dy (G11 - G10))
//        dL/dy   = a * H * ((1 - dx) (G10 - G00) + dx (G11 - G01))
//      and, for the softmax method, dL/dlogit_j = p_j (dL/dp_j - sum_i p_i dL/dp_i).
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
  static __device__ inline void load(const char* p, float (&v)[CV]) {
    const R r = *reinterpret_cast<const R*>(p);
#pragma unroll
    for (int i = 0; i < CV; ++i) v[i] = __uint_as_float(r.w[i]);
  }
  static __device__ inline void store(char* p, const float (&v)[CV]) {
    R r;
#pragma unroll
    for (int i = 0; i < CV; ++i) r.w[i] = __float_as_uint(v[i]);
    *reinterpret_cast<R*>(p) = r;
  }
  static __device__ inline void atomic_add(char* p, const float (&g)[CV], float s) {
#pragma unroll
    for (int i = 0; i < CV; ++i)
      __builtin_amdgcn_global_atomic_fadd_f32(reinterpret_cast<float*>(p) + i, g[i] * s);
  }
};

template <int CV> struct Chan<double, CV> {
  using R = Raw<8 * CV>;
  static __device__ inline void load(const char* p, double (&v)[CV]) {
    const R r = *reinterpret_cast<const R*>(p);
#pragma unroll
    for (int i = 0; i < CV; ++i)
      v[i] = __builtin_bit_cast(double, (uint64_t(r.w[2 * i + 1]) << 32) | r.w[2 * i]);
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
  static __device__ inline void atomic_add(char* p, const double (&g)[CV], double s) {
#pragma unroll
    for (int i = 0; i < CV; ++i)
      __builtin_amdgcn_global_atomic_fadd_f64(reinterpret_cast<double*>(p) + i, g[i] * s);
  }
};

// bf16 and f16 share the packing; only the conversions and the atomic differ.
template <typename T, int CV> struct Chan16 {
  static constexpr bool kBf16 = sizeof(T) == 2 && __is_same(T, bf16_t);
  using R = Raw<2 * CV>;
  static __device__ inline float lo(uint32_t w) { return kBf16 ? bf16_lo(w) : f16_bits(w & 0xffffu); }
  static __device__ inline float hi(uint32_t w) { return kBf16 ? bf16_hi(w) : f16_bits(w >> 16); }
  static __device__ inline uint32_t pack(float a, float b) { return kBf16 ? pack_bf16(a, b) : pack_f16(a, b); }
  static __device__ inline void atomic2(uint32_t* p, uint32_t packed) {
    if constexpr (kBf16)
      __builtin_amdgcn_global_atomic_fadd_v2bf16(reinterpret_cast<bf16x2_v*>(p),
                                                 __builtin_bit_cast(bf16x2_v, packed));
    else
      __builtin_amdgcn_global_atomic_fadd_v2f16(reinterpret_cast<f16x2_v*>(p),
                                                __builtin_bit_cast(f16x2_v, packed));
  }
  static __device__ inline void load(const char* p, float (&v)[CV]) {
    const R r = *reinterpret_cast<const R*>(p);
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
  static __device__ inline void atomic_add(char* p, const float (&g)[CV], float s) {
    if constexpr (CV == 1) {
      // The packed atomic covers the aligned dword; the neighbour gets +0.
      const uintptr_t a = reinterpret_cast<uintptr_t>(p);
      const float x = g[0] * s;
      const uint32_t packed = (a & 2) ? pack(0.0f, x) : pack(x, 0.0f);
      atomic2(reinterpret_cast<uint32_t*>(a & ~uintptr_t(3)), packed);
    } else {
#pragma unroll
      for (int i = 0; i < CV / 2; ++i)
        atomic2(reinterpret_cast<uint32_t*>(p) + i, pack(g[2 * i] * s, g[2 * i + 1] * s));
    }
  }
};
template <int CV> struct Chan<bf16_t, CV> : Chan16<bf16_t, CV> {};
template <int CV> struct Chan<f16_t, CV> : Chan16<f16_t, CV> {};

// ---------------------------------------------------------------------------
// Cross-lane reductions inside the LH lanes of one unit (LH a power of two, the
// unit's lanes contiguous and aligned). Every lane of the wave must call them.

template <typename A> __device__ inline A unit_sum(A v, int lh) {
  for (int m = 1; m < lh; m <<= 1) v += __shfl_xor(v, m, kWave);
  return v;
}
template <typename A> __device__ inline A unit_max(A v, int lh) {
  for (int m = 1; m < lh; m <<= 1) v = fmax(v, __shfl_xor(v, m, kWave));
  return v;
}

__device__ inline float exp_acc(float x) { return __expf(x); }
__device__ inline double exp_acc(double x) { return exp(x); }

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
};

// One pyramid level as the kernels use it. A level whose table entry does not fit
// inside the S positions of the value tensor is marked !ok and sampled nowhere, so
// a malformed table cannot make a kernel read or write outside its tensors.
struct alignas(16) Level {
  int h, w, start, ok;
};

// A staged sample: four corner byte offsets (inside one batch image, with the
// unit's head folded in) and four weights (bilinear * attention, zero for a corner
// outside the level). In the backward the weights slot is reused for the reduced
// G_c once phase 2 has read it.
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

// Geometry of one sample. Contraction is off so that pixel = loc * size - 0.5 and
// the bilinear weights round exactly as the eager reference's separate tensor ops
// do; a fused multiply-add would move samples that sit on a pixel boundary to the
// neighbouring cell and flip their one-sided location gradient.
template <typename A> struct Geom {
  A dx, dy;
  A w00, w01, w10, w11;  // bilinear weights, zero for corners outside the level
  uint32_t off[4];
  bool m00, m01, m10, m11;
};

template <typename A>
__device__ inline Geom<A> geometry(A lx, A ly, const Level lv, uint32_t head_bytes,
                                   uint32_t pos_bytes) {
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
  const bool mx0 = in && ix >= 0, mx1 = in && ix + 1 < lv.w;
  const bool my0 = in && iy >= 0, my1 = in && iy + 1 < lv.h;
  g.m00 = mx0 && my0;
  g.m01 = mx1 && my0;
  g.m10 = mx0 && my1;
  g.m11 = mx1 && my1;
  const int cx0 = max(ix, 0), cx1 = min(ix + 1, lv.w - 1);
  const int cy0 = max(iy, 0), cy1 = min(iy + 1, lv.h - 1);
  const uint32_t base = uint32_t(lv.start) * pos_bytes + head_bytes;
  const uint32_t r0 = uint32_t(cy0 * lv.w), r1 = uint32_t(cy1 * lv.w);
  g.off[0] = base + (r0 + uint32_t(cx0)) * pos_bytes;
  g.off[1] = base + (r0 + uint32_t(cx1)) * pos_bytes;
  g.off[2] = base + (r1 + uint32_t(cx0)) * pos_bytes;
  g.off[3] = base + (r1 + uint32_t(cx1)) * pos_bytes;
  const A one(1);
  g.w00 = g.m00 ? (one - g.dx) * (one - g.dy) : A(0);
  g.w01 = g.m01 ? g.dx * (one - g.dy) : A(0);
  g.w10 = g.m10 ? (one - g.dx) * g.dy : A(0);
  g.w11 = g.m11 ? g.dx * g.dy : A(0);
  return g;
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
  // XCD-aware renumbering: hardware workgroup i runs on XCD i % 8; give XCD x a
  // contiguous range of logical workgroups.
  const int n = p.num_blocks, per = n / kXcds, rem = n % kXcds;
  const int xcd = int(blockIdx.x) % kXcds, slot = int(blockIdx.x) / kXcds;
  const int blk = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
  m.b = blk / p.blocks_per_batch;
  m.unit = (blk - m.b * p.blocks_per_batch) * p.units_per_block + m.wave * m.uw_count + m.uw;
  m.unit_ok = m.unit < p.Q * p.H;
  m.h = m.unit_ok ? m.unit % p.H : 0;
  m.gunit = int64_t(m.b) * p.Q * p.H + m.unit;
  return m;
}

// Phase 1, shared by both directions: stage every sample of the lane's unit and
// return the unit's softmax statistics (max and 1 / sum of exp), if any.
template <typename T, typename TL, bool SOFTMAX>
__device__ inline void stage_samples(const Problem& p, const LaneMap& m, const Level* levels,
                                     Staged<typename Elem<T>::acc>* wst,
                                     typename Elem<T>::acc& smax,
                                     typename Elem<T>::acc& sinv) {
  using A = typename Elem<T>::acc;
  constexpr int ES = Elem<T>::size;
  const int LP = p.L * p.P;
  const TL* loc = reinterpret_cast<const TL*>(p.loc) + m.gunit * LP * 2;
  const T* attn = reinterpret_cast<const T*>(p.attn) + m.gunit * LP;
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
  }
  if (!m.unit_ok) return;
  const uint32_t pos_bytes = uint32_t(p.H * p.D * ES);
  const uint32_t head_bytes = uint32_t(m.h * p.D * ES);
  for (int s = m.t; s < LP; s += m.lh) {
    const Geom<A> g = geometry<A>(load_acc(loc + 2 * s), load_acc(loc + 2 * s + 1),
                                  levels[s / p.P], head_bytes, pos_bytes);
    A a = load_acc(attn + s);
    if constexpr (SOFTMAX) a = exp_acc(a - smax) * sinv;
    Staged<A> st;
#pragma unroll
    for (int c = 0; c < 4; ++c) st.off[c] = g.off[c];
    st.w[0] = g.w00 * a;
    st.w[1] = g.w01 * a;
    st.w[2] = g.w10 * a;
    st.w[3] = g.w11 * a;
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
  Staged<A>* wst = reinterpret_cast<Staged<A>*>(smem + sizeof(Level) * p.L) +
                   m.wave * m.uw_count * LP;

  load_levels(p, levels);
  __syncthreads();
  A smax, sinv;
  stage_samples<T, TL, SOFTMAX>(p, m, levels, wst, smax, sinv);
  __syncthreads();

  if (!m.unit_ok || m.t * CV >= p.D) return;
  const char* img = p.value + int64_t(m.b) * p.S * p.H * p.D * ES;
  const uint32_t lane_bytes = uint32_t(m.t * CV * ES);
  A acc[CV];
#pragma unroll
  for (int i = 0; i < CV; ++i) acc[i] = A(0);
#pragma unroll 2
  for (int s = 0; s < LP; ++s) {
    const Staged<A> st = wst[s * m.uw_count + m.uw];
    A v[4][CV];
#pragma unroll
    for (int c = 0; c < 4; ++c) Chan<T, CV>::load(img + (st.off[c] + lane_bytes), v[c]);
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
// Three kernels on the caller's stream, no atomics to global memory and no buffer
// beyond the three gradients:
//
//   msda_row_summary_kernel    For every (b, h, l) and block of QB queries (QB * P2
//                              = 64 sample slots, P2 = P rounded up to a power of
//                              two), the range of level-l rows its in-bounds
//                              corners touch. Stored, as scratch, at the start of
//                              grad_sampling_locations, which is always large enough
//                              and is written for real only by the third kernel.
//   msda_grad_value_kernel     Owner-computes grad_value: one 1024-thread workgroup
//                              per chunk of NPOS positions of one (b, h) keeps the
//                              chunk's gradient in LDS (fp32; fp64 for double).
//                              Its 16 waves walk the query blocks of every level
//                              that meets the chunk, skip blocks whose row range
//                              misses it, and add a * w_c * grad_out[b, q, h, :] for
//                              the corners inside the chunk with LDS atomics. The
//                              chunk is then written once with plain stores: every
//                              element of grad_value has exactly one writer, so the
//                              result needs no zero-fill, accumulates in fp32 and
//                              does not depend on scheduling beyond fp32 rounding.
//   msda_grad_sample_kernel    Sample-parallel, laid out like the forward: gathers
//                              the four corners of each sample, forms
//                              G_c = <grad_out, value_c>, reduces it across the
//                              unit's lanes and writes grad_loc and grad_attn (the
//                              softmax Jacobian included). Runs last, so it
//                              overwrites the row summaries.

// grad_value, owner-computes, with the chunk accumulator in registers.
//
// Workgroup (b, h, chunk) owns NPOS consecutive positions of grad_value[b, :, h, :].
// Thread t owns the "items" t, t + T, t + 2T, t + 3T (T threads): item i is position
// i / G and channel group i % G (G = D / CVR groups of CVR channels), so the whole
// chunk lives in fp32 (fp64) registers. Per batch of up to one query block per
// wave:
//   A. each wave stages its block's grad_out vectors in LDS and turns every sample
//      of the block into up to four corner records (position in the chunk, query
//      slot, attention * bilinear weight) kept in registers;
//   B. a histogram of the records per position (LDS integer atomics);
//   C. an exclusive scan of the histogram (the start of each position's run);
//   D. each record claims a slot in its position's run (integer atomic) and is
//      stored there;
//   E. each thread walks the runs of the positions it owns and accumulates
//      weight * grad_out into its registers with plain FMAs.
// No floating-point atomics are used: on gfx950 the LDS ones retire at a fraction
// of a lane per clock, while integer LDS atomics run near LDS store rate. Query
// blocks whose row range misses the chunk are never loaded.

constexpr int kGradValueMaxThreads = 1024;
constexpr int kItemsPerThread = 4;
constexpr int kRecordsPerWave = 4 * kWave;

struct GradValuePlan {
  int npos;       // positions per chunk
  int nchunks;    // chunks per (b, h)
  int p2_log2;    // log2 of P rounded up to a power of two
  int nblocks;    // query blocks per (b, h, l): ceil(Q / QB), QB = 64 >> p2_log2
  int groups;     // channel groups per position, G = D / CVR
};

struct alignas(8) RowRange {
  int lo, hi;
};

template <typename A> struct alignas(8) SortedRec {
  A w;
  uint32_t qslot;  // wave * QB + query in block
};

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

// The sample of lane `lane` in block j: (query, point), and whether it exists.
struct BlockSlot {
  int q, pt;
  bool ok;
};
__device__ inline BlockSlot block_slot(const Problem& p, int p2_log2, int j, int lane) {
  BlockSlot bs;
  bs.q = (j << (6 - p2_log2)) + (lane >> p2_log2);
  bs.pt = lane & ((1 << p2_log2) - 1);
  bs.ok = bs.q < p.Q && bs.pt < p.P;
  return bs;
}

// One wave per (b, h, l, block): the range of level-l rows the block's in-bounds
// corners touch (lo > hi when none). Same geometry code and precision as the
// grad_value kernel, so both place every corner in the same row.
template <typename T, typename TL>
__global__ __launch_bounds__(256) void msda_row_summary_kernel(const Problem p, const GradValuePlan gp,
                                                               RowRange* __restrict__ out) {
  using A = typename Elem<T>::acc;
  const int64_t entries = int64_t(p.B) * p.H * p.L * gp.nblocks;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t e = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  if (e >= entries) return;  // uniform per wave
  const int j = int(e % gp.nblocks);
  const int l = int((e / gp.nblocks) % p.L);
  const int h = int((e / (int64_t(gp.nblocks) * p.L)) % p.H);
  const int b = int(e / (int64_t(gp.nblocks) * p.L * p.H));
  int64_t hh, ww, st;
  if (p.index_i32) {
    hh = static_cast<const int32_t*>(p.shapes)[2 * l];
    ww = static_cast<const int32_t*>(p.shapes)[2 * l + 1];
    st = static_cast<const int32_t*>(p.starts)[l];
  } else {
    hh = static_cast<const int64_t*>(p.shapes)[2 * l];
    ww = static_cast<const int64_t*>(p.shapes)[2 * l + 1];
    st = static_cast<const int64_t*>(p.starts)[l];
  }
  const bool ok = hh > 0 && ww > 0 && st >= 0 && hh <= p.S && ww <= p.S && st + hh * ww <= p.S;
  const Level lv = ok ? Level{int(hh), int(ww), int(st), 1} : Level{1, 1, 0, 0};
  const BlockSlot bs = block_slot(p, gp.p2_log2, j, lane);
  int lo = INT32_MAX, hi = INT32_MIN;
  if (bs.ok) {
    const int LP = p.L * p.P;
    const int64_t unit = (int64_t(b) * p.Q + bs.q) * p.H + h;
    const TL* lc = reinterpret_cast<const TL*>(p.loc) + (unit * LP + l * p.P + bs.pt) * 2;
    const Geom<A> g = geometry<A>(load_acc(lc), load_acc(lc + 1), lv, 0u, 1u);
    if (g.m00 || g.m01) lo = hi = (int(g.off[g.m00 ? 0 : 1]) - lv.start) / lv.w;
    if (g.m10 || g.m11) {
      const int r = (int(g.off[g.m10 ? 2 : 3]) - lv.start) / lv.w;
      lo = min(lo, r);
      hi = max(hi, r);
    }
  }
  for (int m = 1; m < kWave; m <<= 1) {
    lo = min(lo, __shfl_xor(lo, m, kWave));
    hi = max(hi, __shfl_xor(hi, m, kWave));
  }
  if (lane == 0) out[e] = RowRange{lo, hi};
}

// Raw (unconverted) element types, so that a prefetch does not wait for its data.
__device__ inline float to_acc(float v) { return v; }
__device__ inline double to_acc(double v) { return v; }
__device__ inline float to_acc(bf16_t v) { return __uint_as_float(uint32_t(v.bits) << 16); }
__device__ inline float to_acc(f16_t v) { return f16_bits(v.bits); }

template <typename TL> struct LocPair {
  TL x, y;
};

// Register copy of what one wave needs from global memory for one query block:
// the lane's location pair and weight, and one 16-byte piece of the block's
// grad_out tile. Kept raw and converted at use, so the loads of the next block stay
// in flight while the current one is processed.
template <typename T, typename TL> struct BlockFetch {
  bool has;
  int j;
  LocPair<TL> loc;
  T a;
  uint4 tv;
};

// Branch-free: every lane issues the same three loads (from clamped, always valid
// addresses) and selects afterwards, so the compiler can count them and leave them in
// flight while the previous block is processed.
template <typename T, typename TL, bool SOFTMAX>
__device__ inline BlockFetch<T, TL> fetch_block(const Problem& p, const GradValuePlan& gp, int sidx,
                                                int nsel, const int* blist, int l, int b, int h,
                                                const TL* loc_all, const T* attn_all, const T* gout,
                                                bool tile_vec) {
  constexpr int kVec = 16 / Elem<T>::size;
  const int lane = threadIdx.x & (kWave - 1);
  BlockFetch<T, TL> f;
  f.has = sidx < nsel;
  // blist[0] is a block of this round only when nsel > 0; otherwise read block 0,
  // which exists whenever the kernel runs (Q > 0). Clamped, so every address below
  // stays inside the tensors whatever the LDS holds.
  const int jj = f.has ? blist[sidx] : (nsel > 0 ? blist[0] : 0);
  f.j = min(max(jj, 0), gp.nblocks - 1);
  const int qb = kWave >> gp.p2_log2;
  const int q0 = f.j * qb;
  const int qn = min(qb, p.Q - q0);
  const BlockSlot bs = block_slot(p, gp.p2_log2, f.j, lane);
  const int LP = p.L * p.P;
  const int q = bs.ok ? bs.q : q0;
  const int s = l * p.P + (bs.ok ? bs.pt : 0);
  const int64_t unit = (int64_t(b) * p.Q + q) * p.H + h;
  f.loc = *reinterpret_cast<const LocPair<TL>*>(loc_all + (unit * LP + s) * 2);
  if constexpr (!SOFTMAX) f.a = attn_all[unit * LP + s];
  else f.a = T{};
  int e = lane * kVec;
  if (!(tile_vec && e < qn * p.D)) e = 0;
  const int qi = e / p.D, c = e - qi * p.D;
  if (tile_vec)
    f.tv = *reinterpret_cast<const uint4*>(gout + ((int64_t(b) * p.Q + q0 + qi) * p.H + h) * p.D + c);
  else
    f.tv = make_uint4(0, 0, 0, 0);
  return f;
}

template <typename T, typename TL, int CVR, bool SOFTMAX>
__global__ __launch_bounds__(kGradValueMaxThreads) void msda_grad_value_kernel(
    const Problem p, const GradValuePlan gp, const RowRange* __restrict__ rows, const int accumulate) {
  using A = typename Elem<T>::acc;
  constexpr int ES = Elem<T>::size;
  extern __shared__ __align__(16) unsigned char smem[];
  const int nthreads = int(blockDim.x), nwaves = nthreads / kWave;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  const int qb = kWave >> gp.p2_log2;
  const int npos = gp.npos;

  // LDS layout; every offset is an integer added to smem, so accesses stay ds_*.
  size_t at = 0;
  Level* levels = reinterpret_cast<Level*>(smem + at);
  at += sizeof(Level) * size_t(p.L);
  SortedRec<A>* sorted = reinterpret_cast<SortedRec<A>*>(smem + at);
  at += sizeof(SortedRec<A>) * size_t(nwaves) * kRecordsPerWave;
  T* gtile = reinterpret_cast<T*>(smem + at);
  at += (sizeof(T) * size_t(nwaves) * qb * p.D + 15) & ~size_t(15);
  int* cnt = reinterpret_cast<int*>(smem + at);
  at += sizeof(int) * size_t(npos);
  int* start = reinterpret_cast<int*>(smem + at);  // npos + 1 entries
  at += sizeof(int) * size_t(npos + 1);
  int* cursor = reinterpret_cast<int*>(smem + at);
  at += sizeof(int) * size_t(npos);
  int* blist = reinterpret_cast<int*>(smem + at);  // selected blocks, one per thread
  at += sizeof(int) * size_t(nthreads);
  int* wave_sums = reinterpret_cast<int*>(smem + at);
  at += (sizeof(int) * size_t(nwaves) + 15) & ~size_t(15);
  LocPair<TL>* sloc = reinterpret_cast<LocPair<TL>*>(smem + at);  // per lane: the staged location
  at += sizeof(LocPair<TL>) * size_t(nthreads);
  T* sattn = reinterpret_cast<T*>(smem + at);  // per lane: the staged weight

  const int n = int(gridDim.x), per = n / kXcds, rem = n % kXcds;
  const int xcd = int(blockIdx.x) % kXcds, slot = int(blockIdx.x) / kXcds;
  const int blk = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
  // Last chunks first: with pyramids stored fine to coarse they hold the coarse,
  // most sampled levels, so the longest workgroups start earliest.
  const int chunk = gp.nchunks - 1 - blk % gp.nchunks;
  const int bh = blk / gp.nchunks;
  const int h = bh % p.H, b = bh / p.H;
  const int p0 = chunk * npos;
  const int p1 = min(p0 + npos, p.S);
  const int LP = p.L * p.P;

  load_levels(p, levels);
  for (int i = tid; i < npos; i += nthreads) cnt[i] = 0;

  A accum[kItemsPerThread][CVR];
#pragma unroll
  for (int k = 0; k < kItemsPerThread; ++k)
#pragma unroll
    for (int c = 0; c < CVR; ++c) accum[k][c] = A(0);
  __syncthreads();

  const T* gout = reinterpret_cast<const T*>(p.grad_out);
  const T* attn_all = reinterpret_cast<const T*>(p.attn);
  const TL* loc_all = reinterpret_cast<const TL*>(p.loc);
  const int P2 = 1 << gp.p2_log2;
  const int tile = qb * p.D;  // elements of one block's grad_out tile
  constexpr int kVec = 16 / ES;
  const bool tile_vec = (p.D % kVec) == 0 && (reinterpret_cast<uintptr_t>(gout) & 15) == 0 &&
                        tile <= kWave * kVec;

  for (int l = 0; l < p.L; ++l) {
    const Level lv = levels[l];
    if (!lv.ok) continue;
    const int a0 = max(p0, lv.start), a1 = min(p1, lv.start + lv.h * lv.w);
    if (a0 >= a1) continue;  // uniform across the workgroup
    const int row_lo = (a0 - lv.start) / lv.w, row_hi = (a1 - 1 - lv.start) / lv.w;
    const RowRange* lrows = rows + ((int64_t(b) * p.H + h) * p.L + l) * gp.nblocks;
    for (int jb = 0; jb < gp.nblocks; jb += nthreads) {
      // Select the blocks of this round whose rows reach the chunk.
      bool reach = false;
      if (jb + tid < gp.nblocks) {
        const RowRange rr = lrows[jb + tid];
        reach = rr.hi >= row_lo && rr.lo <= row_hi;
      }
      int nsel;
      const int at_sel = block_exclusive_scan(reach ? 1 : 0, wave_sums, &nsel);
      if (reach) blist[at_sel] = jb + tid;
      lds_barrier();
      if (nsel == 0) continue;  // uniform across the workgroup
      // Each wave's current block lives in LDS: its lanes' location pairs and
      // weights, and the block's grad_out tile. The next block's global loads are
      // issued at the start of a batch and written to LDS only after the batch's
      // last barrier, so they stay in flight while the batch is processed.
      bool cur_has;
      int cur_j;
      {
        const BlockFetch<T, TL> first = fetch_block<T, TL, SOFTMAX>(p, gp, wave, nsel, blist, l, b, h,
                                                                    loc_all, attn_all, gout, tile_vec);
        sloc[tid] = first.loc;
        sattn[tid] = first.a;
        if (tile_vec && lane * kVec < tile) *reinterpret_cast<uint4*>(gtile + size_t(wave) * tile + lane * kVec) = first.tv;
        cur_has = first.has;
        cur_j = first.j;
      }
      for (int s0 = 0; s0 < nsel; s0 += nwaves) {
        const BlockFetch<T, TL> nxt = fetch_block<T, TL, SOFTMAX>(p, gp, s0 + nwaves + wave, nsel, blist,
                                                                  l, b, h, loc_all, attn_all, gout, tile_vec);
        // A. One block per wave: records in registers (one slot per corner, so the
        // arrays stay in VGPRs).
        bool rv[4] = {false, false, false, false};
        uint32_t rpos[4] = {0u, 0u, 0u, 0u};
        A rw[4] = {A(0), A(0), A(0), A(0)};
        const bool has_block = cur_has;
        const int j = cur_j;
        const int q0 = j * qb;
        const int qn = has_block ? min(qb, p.Q - q0) : 0;
        T* wtile = gtile + size_t(wave) * tile;
        if (has_block) {
          const BlockSlot bs = block_slot(p, gp.p2_log2, j, lane);
          const int s = l * p.P + bs.pt;
          const int64_t unit = (int64_t(b) * p.Q + (bs.q < p.Q ? bs.q : q0)) * p.H + h;
          const LocPair<TL> lp = sloc[tid];
          A a = to_acc(sattn[tid]);
          if (!tile_vec) {
            for (int e = lane; e < qn * p.D; e += kWave) {
              const int qi = e / p.D, c = e - qi * p.D;
              wtile[e] = gout[((int64_t(b) * p.Q + q0 + qi) * p.H + h) * p.D + c];
            }
          }
        if constexpr (SOFTMAX) {
            // The P2 lanes of a query share its L * P logits: max, then sum of exp.
            const T* ua = attn_all + unit * LP;
            A mx = -INFINITY;
            if (bs.q < p.Q)
              for (int i = bs.pt; i < LP; i += P2) mx = fmax(mx, load_acc(ua + i));
            for (int m2 = 1; m2 < P2; m2 <<= 1) mx = fmax(mx, __shfl_xor(mx, m2, kWave));
            A sum(0);
            if (bs.q < p.Q)
              for (int i = bs.pt; i < LP; i += P2) sum += exp_acc(load_acc(ua + i) - mx);
            for (int m2 = 1; m2 < P2; m2 <<= 1) sum += __shfl_xor(sum, m2, kWave);
            if (bs.ok) a = exp_acc(load_acc(ua + s) - mx) / sum;
          }
          if (bs.ok) {
            const Geom<A> g = geometry<A>(to_acc(lp.x), to_acc(lp.y), lv, 0u, 1u);
            const bool m[4] = {g.m00, g.m01, g.m10, g.m11};
            const A wb[4] = {g.w00, g.w01, g.w10, g.w11};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              rv[c] = m[c] && int(g.off[c]) >= a0 && int(g.off[c]) < a1;
              rpos[c] = g.off[c] - uint32_t(p0);
              rw[c] = wb[c] * a;
            }
          }
        }
        // B. Histogram.
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (rv[c]) atomicAdd(&cnt[rpos[c]], 1);
        lds_barrier();
        // C. Start of every position's run.
        {
          int total;
          const int v = tid < npos ? cnt[tid] : 0;
          const int ex = block_exclusive_scan(v, wave_sums, &total);
          if (tid < npos) {
            start[tid] = ex;
            cursor[tid] = ex;
          }
          if (tid == 0) start[npos] = total;
        }
        lds_barrier();
        // D. Place the records.
        const uint32_t qslot = uint32_t(wave * qb + (lane >> gp.p2_log2));
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (rv[c]) {
            const int dst = atomicAdd(&cursor[rpos[c]], 1);
            sorted[dst] = SortedRec<A>{rw[c], qslot};
          }
        }
        lds_barrier();
        // E. Accumulate the runs of the owned items.
#pragma unroll
        for (int k = 0; k < kItemsPerThread; ++k) {
          const int item = tid + k * nthreads;
          const int pos = item / gp.groups, grp = item - pos * gp.groups;
          if (pos < npos) {
            const int r1 = start[pos + 1];
            for (int r = start[pos]; r < r1; ++r) {
              const SortedRec<A> rec = sorted[r];
              const T* gq = gtile + size_t(rec.qslot) * p.D + grp * CVR;
              A gv[CVR];
              Chan<T, CVR>::load(reinterpret_cast<const char*>(gq), gv);
#pragma unroll
              for (int c = 0; c < CVR; ++c) accum[k][c] = fma(rec.w, gv[c], accum[k][c]);
            }
          }
        }
        for (int i = tid; i < npos; i += nthreads) cnt[i] = 0;
        lds_barrier();
        sloc[tid] = nxt.loc;
        sattn[tid] = nxt.a;
        if (tile_vec && lane * kVec < tile) *reinterpret_cast<uint4*>(wtile + lane * kVec) = nxt.tv;
        cur_has = nxt.has;
        cur_j = nxt.j;
      }
    }
  }

  // Write the owned items: the only writer of these grad_value elements.
  T* gv_out = reinterpret_cast<T*>(p.grad_value);
  const int64_t img = int64_t(b) * p.S * p.H * p.D;
#pragma unroll
  for (int k = 0; k < kItemsPerThread; ++k) {
    const int item = tid + k * nthreads;
    const int pos = item / gp.groups, grp = item - pos * gp.groups;
    if (pos < p1 - p0) {
      char* dst = reinterpret_cast<char*>(gv_out + img + (int64_t(p0 + pos) * p.H + h) * p.D + grp * CVR);
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

  load_levels(p, levels);
  __syncthreads();
  A smax, sinv;
  stage_samples<T, TL, SOFTMAX>(p, m, levels, wst, smax, sinv);
  __syncthreads();

  // Gather the corners and form G_c; the lane that staged sample s keeps its G_c
  // in the sample's slot.
  const bool lane_ok = m.unit_ok && m.t * CV < p.D;
  const char* img = p.value + int64_t(m.b) * p.S * p.H * p.D * ES;
  const uint32_t lane_bytes = uint32_t(m.t * CV * ES);
  A g[CV];
  if (lane_ok) {
    Chan<T, CV>::load(p.grad_out + (m.gunit * p.D + m.t * CV) * ES, g);
  } else {
#pragma unroll
    for (int i = 0; i < CV; ++i) g[i] = A(0);
  }
  for (int s = 0; s < LP; ++s) {
    Staged<A>* slot = wst + s * m.uw_count + m.uw;
    const Staged<A> st = *slot;
    A G[4] = {A(0), A(0), A(0), A(0)};
    if (lane_ok) {
      A v[4][CV];
#pragma unroll
      for (int c = 0; c < 4; ++c) Chan<T, CV>::load(img + (st.off[c] + lane_bytes), v[c]);
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int i = 0; i < CV; ++i) G[c] = fma(g[i], v[c][i], G[c]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) G[c] = unit_sum(G[c], m.lh);
    if (m.unit_ok && m.t == (s & (m.lh - 1))) {
#pragma unroll
      for (int c = 0; c < 4; ++c) slot->w[c] = G[c];
    }
  }

  // Per-sample location and weight gradients by the lane that staged the sample.
  const TL* loc = reinterpret_cast<const TL*>(p.loc) + m.gunit * LP * 2;
  const T* attn = reinterpret_cast<const T*>(p.attn) + m.gunit * LP;
  TL* gloc = reinterpret_cast<TL*>(p.grad_loc) + m.gunit * LP * 2;
  T* gattn = reinterpret_cast<T*>(p.grad_attn) + m.gunit * LP;
  const uint32_t pos_bytes = uint32_t(p.H * p.D * ES);
  const uint32_t head_bytes = uint32_t(m.h * p.D * ES);
  A dot(0);
  if (m.unit_ok) {
    for (int s = m.t; s < LP; s += m.lh) {
      const Level lv = levels[s / p.P];
      const Geom<A> ge = geometry<A>(load_acc(loc + 2 * s), load_acc(loc + 2 * s + 1), lv,
                                     head_bytes, pos_bytes);
      A a = load_acc(attn + s);
      if constexpr (SOFTMAX) a = exp_acc(a - smax) * sinv;
      Staged<A>* slot = wst + s * m.uw_count + m.uw;
      const A G00 = ge.m00 ? slot->w[0] : A(0);
      const A G01 = ge.m01 ? slot->w[1] : A(0);
      const A G10 = ge.m10 ? slot->w[2] : A(0);
      const A G11 = ge.m11 ? slot->w[3] : A(0);
      const A one(1);
      const A gpv = ge.w00 * G00 + ge.w01 * G01 + ge.w10 * G10 + ge.w11 * G11;
      const A gx = a * A(lv.w) * ((one - ge.dy) * (G01 - G00) + ge.dy * (G11 - G10));
      const A gy = a * A(lv.h) * ((one - ge.dx) * (G10 - G00) + ge.dx * (G11 - G01));
      store_elem(gloc + 2 * s, gx);
      store_elem(gloc + 2 * s + 1, gy);
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
              int64_t P, bool backward, const void* const* vec_ptrs, int n_vec, Plan* plan) {
  const int es = elem_size(dtype);
  if (es == 0) return fail(MSDA_ERR_INVALID, "msda: unknown value dtype code %d", dtype);
  if (B < 0 || S < 0 || H < 0 || D < 0 || Q < 0 || L < 0 || P < 0)
    return fail(MSDA_ERR_INVALID, "msda: negative size (B=%lld S=%lld H=%lld D=%lld Q=%lld L=%lld P=%lld)",
                (long long)B, (long long)S, (long long)H, (long long)D, (long long)Q,
                (long long)L, (long long)P);
  if (H == 0 || D == 0 || L == 0 || P == 0)
    return fail(MSDA_ERR_INVALID, "msda: heads, channels, levels and points must be positive");
  const int64_t kInt32 = 2147483647;
  if (S * H * D * es >= kInt32)
    return fail(MSDA_ERR_UNSUPPORTED,
                "msda: one batch image of value holds %lld bytes; the kernels address an image "
                "with 32-bit offsets and take at most 2^31 - 1 bytes",
                (long long)(S * H * D * es));
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
  const int uw = kWave >> lh_log2;
  const size_t staged = (dtype == MSDA_F64) ? sizeof(Staged<double>) : sizeof(Staged<float>);
  const size_t per_wave = size_t(uw) * size_t(L * P) * staged;
  const size_t levels_bytes = sizeof(Level) * size_t(L);
  if (levels_bytes + per_wave > kMaxLds)
    return fail(MSDA_ERR_UNSUPPORTED,
                "msda: %lld samples per (query, head) do not fit the %zu-byte LDS staging of one "
                "wave (%zu bytes needed)",
                (long long)(L * P), kMaxLds, levels_bytes + per_wave);
  const int64_t units = Q * H;
  int waves = kMaxWavesPerBlock;
  // Fewer waves per workgroup when the grid would leave CUs idle or LDS is short.
  while (waves > 1) {
    const int64_t blocks = B * ((units + int64_t(waves) * uw - 1) / (int64_t(waves) * uw));
    if (levels_bytes + per_wave * waves <= kMaxLds && blocks >= 2048) break;
    waves >>= 1;
  }
  (void)backward;
  plan->cv = cv;
  plan->lh_log2 = lh_log2;
  plan->waves = waves;
  plan->units_per_block = waves * uw;
  plan->blocks_per_batch = int((units + plan->units_per_block - 1) / plan->units_per_block);
  plan->num_blocks = B * plan->blocks_per_batch;
  plan->lds = levels_bytes + per_wave * waves;
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

// Launch layout of the backward's three kernels.
struct BackwardPlan {
  GradValuePlan gv;
  int gv_threads;
  int cvr;
  size_t gv_lds;
  int64_t gv_blocks;
  int64_t summary_entries;
  Plan sample;
};

size_t device_lds_limit() {
  int dev = 0, bytes = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
      bytes <= 0)
    return 64 * 1024;
  return size_t(bytes);
}

size_t grad_value_lds(int dtype, int threads, int64_t L, int64_t D, int qb, int64_t npos) {
  const size_t es = size_t(elem_size(dtype));
  const size_t rec = dtype == MSDA_F64 ? sizeof(SortedRec<double>) : sizeof(SortedRec<float>);
  const size_t waves = size_t(threads / kWave);
  size_t at = sizeof(Level) * size_t(L);
  at += rec * waves * kRecordsPerWave;
  at += (es * waves * size_t(qb) * size_t(D) + 15) & ~size_t(15);
  at += sizeof(int) * (3 * size_t(npos) + 1);
  at += sizeof(int) * size_t(threads);
  at += (sizeof(int) * waves + 15) & ~size_t(15);
  at += (dtype == MSDA_F64 ? 16 : 8) * size_t(threads);  // staged location pairs (widest case)
  at += es * size_t(threads);                            // staged weights
  return at;
}

int make_backward_plan(int dtype, int64_t B, int64_t S, int64_t H, int64_t D, int64_t Q, int64_t L,
                       int64_t P, int loc_dtype, const void* const* vec_ptrs, int n_vec,
                       size_t lds_limit, BackwardPlan* plan) {
  int rc = make_plan(dtype, B, S, H, D, Q, L, P, true, vec_ptrs, n_vec, &plan->sample);
  if (rc != MSDA_OK) return rc;
  if (P > kWave)
    return fail(MSDA_ERR_UNSUPPORTED, "msda: the backward takes at most %d points per level", kWave);
  int p2_log2 = 0;
  while ((int64_t(1) << p2_log2) < P) ++p2_log2;
  const int qb = kWave >> p2_log2;
  const int64_t nblocks = (Q + qb - 1) / qb;
  const int64_t entries = B * H * L * nblocks;
  const int64_t loc_bytes = B * Q * H * L * P * 2 * elem_size(loc_dtype);
  if (entries * int64_t(sizeof(RowRange)) > loc_bytes)
    return fail(MSDA_ERR_UNSUPPORTED, "msda: row summaries do not fit the location gradient");
  // Channels per register item: the widest power of two that divides D, fits a
  // 16-byte access and keeps grad_value aligned to it.
  const int es = elem_size(dtype);
  int cvr = 16 / es;
  while (cvr > 1) {
    bool ok = D % cvr == 0;
    for (int i = 0; i < n_vec && ok; ++i) ok = aligned(vec_ptrs[i], cvr * es);
    if (ok) break;
    cvr >>= 1;
  }
  const int64_t groups = D / cvr;
  const size_t budget = lds_limit < 160 * 1024 ? lds_limit : 160 * 1024;
  int threads = kGradValueMaxThreads;
  int64_t npos = 0;
  for (;;) {
    npos = std::min<int64_t>({int64_t(threads), int64_t(threads) * kItemsPerThread / groups, S});
    if (npos >= 1 && grad_value_lds(dtype, threads, L, D, qb, npos) <= budget) break;
    if (threads == kWave)
      return fail(MSDA_ERR_UNSUPPORTED,
                  "msda: %lld channels per head do not fit the backward's register and LDS budget",
                  (long long)D);
    threads >>= 1;
  }
  const int64_t nchunks = (S + npos - 1) / npos;
  const int64_t blocks = B * H * nchunks;
  if (blocks >= 2147483647 || nblocks >= 2147483647 || entries * kWave >= (int64_t(1) << 40))
    return fail(MSDA_ERR_UNSUPPORTED, "msda: backward grid too large");
  plan->gv = GradValuePlan{int(npos), int(nchunks), p2_log2, int(nblocks), int(groups)};
  plan->gv_threads = threads;
  plan->cvr = cvr;
  plan->gv_lds = grad_value_lds(dtype, threads, L, D, qb, npos);
  plan->gv_blocks = blocks;
  plan->summary_entries = entries;
  return MSDA_OK;
}

template <typename T, typename TL, bool SOFTMAX>
hipError_t launch_grad_value(const BackwardPlan& plan, const Problem& p, const RowRange* rows,
                             int accumulate, hipStream_t st) {
  constexpr int kMaxCv = 16 / Elem<T>::size;
  const void* fn = nullptr;
  switch (plan.cvr) {
    case 1: fn = reinterpret_cast<const void*>(msda_grad_value_kernel<T, TL, 1, SOFTMAX>); break;
    case 2: fn = reinterpret_cast<const void*>(msda_grad_value_kernel<T, TL, 2, SOFTMAX>); break;
    case 4:
      if constexpr (kMaxCv >= 4) fn = reinterpret_cast<const void*>(msda_grad_value_kernel<T, TL, 4, SOFTMAX>);
      break;
    case 8:
      if constexpr (kMaxCv >= 8) fn = reinterpret_cast<const void*>(msda_grad_value_kernel<T, TL, 8, SOFTMAX>);
      break;
  }
  if (!fn) return hipErrorInvalidValue;
  if (plan.gv_lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(plan.gv_lds));
    if (e != hipSuccess) return e;
  }
  const dim3 grid(unsigned(plan.gv_blocks)), block(unsigned(plan.gv_threads));
  switch (plan.cvr) {
    case 1:
      hipLaunchKernelGGL((msda_grad_value_kernel<T, TL, 1, SOFTMAX>), grid, block, plan.gv_lds, st, p,
                         plan.gv, rows, accumulate);
      break;
    case 2:
      hipLaunchKernelGGL((msda_grad_value_kernel<T, TL, 2, SOFTMAX>), grid, block, plan.gv_lds, st, p,
                         plan.gv, rows, accumulate);
      break;
    case 4:
      if constexpr (kMaxCv >= 4)
        hipLaunchKernelGGL((msda_grad_value_kernel<T, TL, 4, SOFTMAX>), grid, block, plan.gv_lds, st, p,
                           plan.gv, rows, accumulate);
      break;
    case 8:
      if constexpr (kMaxCv >= 8)
        hipLaunchKernelGGL((msda_grad_value_kernel<T, TL, 8, SOFTMAX>), grid, block, plan.gv_lds, st, p,
                           plan.gv, rows, accumulate);
      break;
  }
  return hipGetLastError();
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

}  // namespace

extern "C" {

const char* msda_last_error(void) { return g_last_error; }

int msda_abi_version(void) { return MSDA_ABI_VERSION; }

int msda_launch_geometry(int value_dtype, int64_t batch, int64_t spatial, int64_t heads,
                         int64_t channels, int64_t queries, int64_t levels, int64_t points,
                         int backward, int* channels_per_lane, int* lanes_per_unit,
                         int* waves_per_block, int64_t* num_blocks) {
  if (elem_size(value_dtype) == 0)
    return fail(MSDA_ERR_INVALID, "msda: unknown value dtype code %d", value_dtype);
  if (backward) {
    BackwardPlan bp;
    const int rc = make_backward_plan(value_dtype, batch, spatial, heads, channels, queries,
                                      levels, points, value_dtype, nullptr, 0, 160 * 1024, &bp);
    if (rc != MSDA_OK) return rc;
    // The grad_value kernel's layout: channels per register item, positions per
    // chunk, waves per workgroup and workgroups.
    if (channels_per_lane) *channels_per_lane = bp.cvr;
    if (lanes_per_unit) *lanes_per_unit = bp.gv.npos;
    if (waves_per_block) *waves_per_block = bp.gv_threads / kWave;
    if (num_blocks) *num_blocks = bp.gv_blocks;
    return MSDA_OK;
  }
  Plan plan;
  const int rc = make_plan(value_dtype, batch, spatial, heads, channels, queries, levels, points,
                           false, nullptr, 0, &plan);
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
                 vec, 2, &plan);
  if (rc != MSDA_OK) return rc;
  Problem p = make_problem(value, spatial_shapes, level_start_index, index_dtype,
                           sampling_locations, attention_weights, batch, spatial, heads,
                           channels, queries, levels, points, plan);
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

int msda_backward(const void* value, int value_dtype, const void* spatial_shapes,
                  const void* level_start_index, int index_dtype, const void* sampling_locations,
                  int loc_dtype, const void* attention_weights, const void* grad_output,
                  void* grad_value, void* grad_sampling_locations, void* grad_attention_weights,
                  int64_t batch, int64_t spatial, int64_t heads, int64_t channels,
                  int64_t queries, int64_t levels, int64_t points, int flags, void* stream) {
  g_last_error[0] = '\0';
  int rc = check_call(value_dtype, index_dtype, loc_dtype, batch, spatial, heads, channels,
                      queries, levels, points, flags, MSDA_SOFTMAX | MSDA_ACCUMULATE_GRAD_VALUE);
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
  if (reinterpret_cast<uintptr_t>(grad_sampling_locations) % alignof(RowRange) != 0)
    return fail(MSDA_ERR_INVALID, "msda_backward: grad_sampling_locations must be 4-byte aligned");
  const void* vec[] = {value, grad_output, grad_value};
  BackwardPlan plan;
  rc = make_backward_plan(value_dtype, batch, spatial, heads, channels, queries, levels, points,
                          loc_dtype, vec, 2, device_lds_limit(), &plan);
  if (rc != MSDA_OK) return rc;
  Problem p = make_problem(value, spatial_shapes, level_start_index, index_dtype,
                           sampling_locations, attention_weights, batch, spatial, heads,
                           channels, queries, levels, points, plan.sample);
  p.grad_out = static_cast<const char*>(grad_output);
  p.grad_value = static_cast<char*>(grad_value);
  p.grad_loc = static_cast<char*>(grad_sampling_locations);
  p.grad_attn = static_cast<char*>(grad_attention_weights);
  RowRange* rows = static_cast<RowRange*>(grad_sampling_locations);
  const bool softmax = flags & MSDA_SOFTMAX;
  const hipError_t err = dispatch(
      value_dtype, loc_dtype == MSDA_F32 && value_dtype != MSDA_F32, plan.sample.cv,
      [&]<typename T, typename TL, int CV>() {
        const unsigned summary_blocks = unsigned((plan.summary_entries * kWave + 255) / 256);
        hipLaunchKernelGGL((msda_row_summary_kernel<T, TL>), dim3(summary_blocks), dim3(256), 0, st,
                           p, plan.gv, rows);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        e = softmax ? launch_grad_value<T, TL, true>(plan, p, rows, int(accumulate), st)
                    : launch_grad_value<T, TL, false>(plan, p, rows, int(accumulate), st);
        if (e != hipSuccess) return e;
        const dim3 grid(unsigned(plan.sample.num_blocks)), block(unsigned(kWave * plan.sample.waves));
        if (softmax)
          hipLaunchKernelGGL((msda_grad_sample_kernel<T, TL, CV, true>), grid, block,
                             plan.sample.lds, st, p);
        else
          hipLaunchKernelGGL((msda_grad_sample_kernel<T, TL, CV, false>), grid, block,
                             plan.sample.lds, st, p);
        return hipGetLastError();
      });
  if (err != hipSuccess)
    return fail(MSDA_ERR_HIP, "msda_backward: launch failed: %s", hipGetErrorString(err));
  return MSDA_OK;
}

}  // extern "C"
