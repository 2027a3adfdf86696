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

template <typename T, typename TL, int CV, bool SOFTMAX>
__global__ __launch_bounds__(kWave * kMaxWavesPerBlock) void msda_backward_kernel(const Problem p) {
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

  // Phase 2: gather, corner dot products, atomic scatter into grad_value.
  const bool lane_ok = m.unit_ok && m.t * CV < p.D;
  const int64_t img_off = int64_t(m.b) * p.S * p.H * p.D * ES;
  const char* img = p.value + img_off;
  char* gimg = p.grad_value + img_off;
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
    if (lane_ok) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (st.w[c] != A(0)) Chan<T, CV>::atomic_add(gimg + (st.off[c] + lane_bytes), g, st.w[c]);
    }
  }

  // Phase 3: per-sample location and weight gradients, by the lane that staged
  // the sample (it alone wrote the sample's G_c back into its slot).
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
      const A gp = ge.w00 * G00 + ge.w01 * G01 + ge.w10 * G10 + ge.w11 * G11;
      const A gx = a * A(lv.w) * ((one - ge.dy) * (G01 - G00) + ge.dy * (G11 - G10));
      const A gy = a * A(lv.h) * ((one - ge.dx) * (G10 - G00) + ge.dx * (G11 - G01));
      store_elem(gloc + 2 * s, gx);
      store_elem(gloc + 2 * s + 1, gy);
      if constexpr (SOFTMAX) {
        dot += a * gp;
        slot->w[0] = gp;
      } else {
        store_elem(gattn + s, gp);
      }
    }
  }
  if constexpr (SOFTMAX) {
    dot = unit_sum(dot, m.lh);
    if (m.unit_ok) {
      for (int s = m.t; s < LP; s += m.lh) {
        const A a = exp_acc(load_acc(attn + s) - smax) * sinv;
        const A gp = wst[s * m.uw_count + m.uw].w[0];
        store_elem(gattn + s, a * (gp - dot));
      }
    }
  }
}

// Zero-fill of grad_value before the atomics: a plain kernel (not hipMemsetAsync),
// so a caller may capture the backward in a HIP graph.
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

template <bool BWD, typename T, typename TL, int CV>
hipError_t launch_cv(const Problem& p, const Plan& plan, int softmax, hipStream_t stream) {
  const dim3 grid(unsigned(plan.num_blocks)), block(unsigned(kWave * plan.waves));
  if constexpr (BWD) {
    if (softmax)
      hipLaunchKernelGGL((msda_backward_kernel<T, TL, CV, true>), grid, block, plan.lds, stream, p);
    else
      hipLaunchKernelGGL((msda_backward_kernel<T, TL, CV, false>), grid, block, plan.lds, stream, p);
  } else {
    if (softmax)
      hipLaunchKernelGGL((msda_forward_kernel<T, TL, CV, true>), grid, block, plan.lds, stream, p);
    else
      hipLaunchKernelGGL((msda_forward_kernel<T, TL, CV, false>), grid, block, plan.lds, stream, p);
  }
  return hipGetLastError();
}

template <bool BWD, typename T, typename TL>
hipError_t launch_tl(const Problem& p, const Plan& plan, int softmax, hipStream_t stream) {
  constexpr int kMaxCv = 16 / Elem<T>::size;
  switch (plan.cv) {
    case 1: return launch_cv<BWD, T, TL, 1>(p, plan, softmax, stream);
    case 2: return launch_cv<BWD, T, TL, 2>(p, plan, softmax, stream);
    case 4:
      if constexpr (kMaxCv >= 4) return launch_cv<BWD, T, TL, 4>(p, plan, softmax, stream);
      break;
    case 8:
      if constexpr (kMaxCv >= 8) return launch_cv<BWD, T, TL, 8>(p, plan, softmax, stream);
      break;
  }
  return hipErrorInvalidValue;
}

template <bool BWD, typename T>
hipError_t launch_t(const Problem& p, const Plan& plan, int loc_f32, int softmax, hipStream_t stream) {
  if constexpr (__is_same(T, float) || __is_same(T, double)) {
    return launch_tl<BWD, T, T>(p, plan, softmax, stream);
  } else {
    return loc_f32 ? launch_tl<BWD, T, float>(p, plan, softmax, stream)
                   : launch_tl<BWD, T, T>(p, plan, softmax, stream);
  }
}

template <bool BWD>
hipError_t launch(int dtype, const Problem& p, const Plan& plan, int loc_f32, int softmax,
                  hipStream_t stream) {
  switch (dtype) {
    case MSDA_F32: return launch_t<BWD, float>(p, plan, loc_f32, softmax, stream);
    case MSDA_F64: return launch_t<BWD, double>(p, plan, loc_f32, softmax, stream);
    case MSDA_BF16: return launch_t<BWD, bf16_t>(p, plan, loc_f32, softmax, stream);
    case MSDA_F16: return launch_t<BWD, f16_t>(p, plan, loc_f32, softmax, stream);
  }
  return hipErrorInvalidValue;
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
  Plan plan;
  const int rc = make_plan(value_dtype, batch, spatial, heads, channels, queries, levels, points,
                           backward != 0, nullptr, 0, &plan);
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
  const hipError_t err = launch<false>(value_dtype, p, plan, loc_dtype == MSDA_F32,
                                       flags & MSDA_SOFTMAX, st);
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
  (void)hipGetLastError();
  if (value_bytes > 0 && !(flags & MSDA_ACCUMULATE_GRAD_VALUE)) {
    rc = zero_fill(grad_value, value_bytes, st, "msda_backward");
    if (rc != MSDA_OK) return rc;
  }
  if (sample_count == 0) return MSDA_OK;
  if (channels == 0 || spatial == 0) {
    // Nothing to sample from: every location and weight gradient is zero.
    rc = zero_fill(grad_sampling_locations, sample_count * 2 * elem_size(loc_dtype), st,
                   "msda_backward");
    if (rc != MSDA_OK) return rc;
    return zero_fill(grad_attention_weights, sample_count * es, st, "msda_backward");
  }
  if (!value || !spatial_shapes || !level_start_index || !sampling_locations ||
      !attention_weights || !grad_output)
    return fail(MSDA_ERR_INVALID, "msda_backward: null input tensor pointer");
  const void* vec[] = {value, grad_output, grad_value};
  Plan plan;
  rc = make_plan(value_dtype, batch, spatial, heads, channels, queries, levels, points, true,
                 vec, 3, &plan);
  if (rc != MSDA_OK) return rc;
  Problem p = make_problem(value, spatial_shapes, level_start_index, index_dtype,
                           sampling_locations, attention_weights, batch, spatial, heads,
                           channels, queries, levels, points, plan);
  p.grad_out = static_cast<const char*>(grad_output);
  p.grad_value = static_cast<char*>(grad_value);
  p.grad_loc = static_cast<char*>(grad_sampling_locations);
  p.grad_attn = static_cast<char*>(grad_attention_weights);
  const hipError_t err = launch<true>(value_dtype, p, plan, loc_dtype == MSDA_F32,
                                      flags & MSDA_SOFTMAX, st);
  if (err != hipSuccess)
    return fail(MSDA_ERR_HIP, "msda_backward: launch failed: %s", hipGetErrorString(err));
  return MSDA_OK;
}

}  // extern "C"
