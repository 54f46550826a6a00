// Optimizer-path kernels: fused AdamW over a flat fp32 master, gradient
// sum-of-squares and clip factor, fills, casts, accumulates, and the
// multi-tensor gather/scatter between per-parameter storages and flat buffers.
//
// All are HBM-bound streaming kernels: 16-byte vector accesses where the
// pointers allow it; AdamW runs one 4-element group per thread with
// non-temporal accesses, the others grid-stride loops sized to a few waves of
// workgroups per compute unit.
#include <algorithm>

#include "lz_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kFillF64 = 3;  // lz_fill's code for float64 (the norm accumulators)

inline int stream_grid(int64_t work_items) {
  int64_t blocks = lz_cdiv(work_items, kThreads);
  int64_t cap = (int64_t)lz_num_cus() * 8;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  return (int)blocks;
}

struct AdamArgs {
  float beta1, beta2;
  float omb1, omb2;     // 1 - beta1, 1 - beta2
  float wd_factor;      // 1 - lr * weight_decay
  float sqrt_bc2;       // sqrt(1 - beta2^t)
  float eps;
  float neg_step;       // -lr / (1 - beta1^t)
  int apply_wd;
};

// One AdamW element update, in the operation order of the reference update
// (zero/stage0_ddp.py:73-88): moments, decoupled decay, then the
// bias-corrected step.
__device__ __forceinline__ void adam_elem(float& p, float& m, float& v, float g, const AdamArgs& a) {
  m = fmaf(a.omb1, g, m * a.beta1);
  v = fmaf(a.omb2 * g, g, v * a.beta2);
  if (a.apply_wd) p = p * a.wd_factor;
  const float denom = sqrtf(v) / a.sqrt_bc2 + a.eps;
  p = fmaf(a.neg_step, m / denom, p);
}

// The step-dependent factors from device memory (written by
// adamw_step_kernel) when `hyper` is set: -lr/bc1, sqrt(bc2), 1 - lr*wd.
__device__ __forceinline__ AdamArgs with_hyper(AdamArgs a, const float* hyper) {
  if (hyper) {
    a.neg_step = hyper[0];
    a.sqrt_bc2 = hyper[1];
    a.wd_factor = hyper[2];
  }
  return a;
}

template <typename G, typename PO>
__global__ void __launch_bounds__(kThreads) adamw_scalar_kernel(float* __restrict__ p, float* __restrict__ m,
                                                                 float* __restrict__ v, const G* __restrict__ g,
                                                                 PO* __restrict__ pout, int64_t n, AdamArgs a0,
                                                                 const float* __restrict__ scale_ptr,
                                                                 const float* __restrict__ hyper) {
  const AdamArgs a = with_hyper(a0, hyper);
  const float scale = scale_ptr ? *scale_ptr : 1.0f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float pp = p[i], mm = m[i], vv = v[i];
    float gg = Elem<G>::load(g, i);
    if (scale_ptr) gg = gg * scale;
    adam_elem(pp, mm, vv, gg, a);
    p[i] = pp;
    m[i] = mm;
    v[i] = vv;
    if (pout) Elem<PO>::store(pout, i, pp);
  }
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// 4-element vector accesses.  The streaming optimizer kernels touch each byte
// once, so their accesses are non-temporal (they do not displace the caches'
// contents), which measured faster on MI355X.
template <typename T>
struct Vec4;
template <>
struct Vec4<float> {
  static __device__ __forceinline__ void load(const float* p, int64_t i, float (&r)[4]) {
    const f32x4_t x = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p + i));
    r[0] = x[0]; r[1] = x[1]; r[2] = x[2]; r[3] = x[3];
  }
  static __device__ __forceinline__ void store(float* p, int64_t i, const float (&r)[4]) {
    const f32x4_t x = {r[0], r[1], r[2], r[3]};
    __builtin_nontemporal_store(x, reinterpret_cast<f32x4_t*>(p + i));
  }
};
template <>
struct Vec4<uint16_t> {
  static __device__ __forceinline__ void load(const uint16_t* p, int64_t i, float (&r)[4]) {
    const u32x2_t x = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p + i));
    r[0] = bf2f(x[0] & 0xffff); r[1] = bf2f(x[0] >> 16); r[2] = bf2f(x[1] & 0xffff); r[3] = bf2f(x[1] >> 16);
  }
  static __device__ __forceinline__ void store(uint16_t* p, int64_t i, const float (&r)[4]) {
    const u32x2_t x = {(uint32_t)f2bf(r[0]) | ((uint32_t)f2bf(r[1]) << 16),
                       (uint32_t)f2bf(r[2]) | ((uint32_t)f2bf(r[3]) << 16)};
    __builtin_nontemporal_store(x, reinterpret_cast<u32x2_t*>(p + i));
  }
};
template <>
struct Vec4<_Float16> {
  static __device__ __forceinline__ void load(const _Float16* p, int64_t i, float (&r)[4]) {
    const u32x2_t x = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p + i));
    r[0] = h2f(x[0] & 0xffff); r[1] = h2f(x[0] >> 16); r[2] = h2f(x[1] & 0xffff); r[3] = h2f(x[1] >> 16);
  }
  static __device__ __forceinline__ void store(_Float16* p, int64_t i, const float (&r)[4]) {
    const u32x2_t x = {pack_f16x2(r[0], r[1]), pack_f16x2(r[2], r[3])};
    __builtin_nontemporal_store(x, reinterpret_cast<u32x2_t*>(p + i));
  }
};

// One 4-element group per thread over the whole array (a full grid measured
// faster than a grid-stride loop: consecutive workgroups stream consecutive
// memory); the n % 4 tail goes to the scalar kernel.
constexpr int kAdamThreads = 128;

// `part` (optional): one float64 per workgroup, the sum of the squares of the
// gradient values it read (before the clip scale), for a step that reports
// the norm without clipping: the norm then costs no pass of its own.
template <typename G, typename PO>
__global__ void __launch_bounds__(kAdamThreads) adamw_vec_kernel(float* __restrict__ p, float* __restrict__ m,
                                                                  float* __restrict__ v, const G* __restrict__ g,
                                                                  PO* __restrict__ pout, int64_t n4, AdamArgs a0,
                                                                  const float* __restrict__ scale_ptr,
                                                                  const float* __restrict__ hyper,
                                                                  double* __restrict__ part) {
  const int64_t q = (int64_t)blockIdx.x * kAdamThreads + threadIdx.x;
  float gg[4] = {0.f, 0.f, 0.f, 0.f};
  if (q < n4) {
    const AdamArgs a = with_hyper(a0, hyper);
    const int64_t i = q << 2;
    float pp[4], mm[4], vv[4];
    Vec4<float>::load(p, i, pp);
    Vec4<float>::load(m, i, mm);
    Vec4<float>::load(v, i, vv);
    Vec4<G>::load(g, i, gg);
    const float scale = scale_ptr ? *scale_ptr : 1.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float gj = scale_ptr ? gg[j] * scale : gg[j];
      adam_elem(pp[j], mm[j], vv[j], gj, a);
    }
    Vec4<float>::store(p, i, pp);
    Vec4<float>::store(m, i, mm);
    Vec4<float>::store(v, i, vv);
    if (pout) Vec4<PO>::store(pout, i, pp);
  }
  if (part) {
    // every thread joins (those past the end with zeros), after its stores
    // are issued; the barrier orders LDS only, so it does not wait for them
    __shared__ double red[kAdamThreads / 64];
    const float sq = fmaf(gg[0], gg[0], fmaf(gg[1], gg[1], fmaf(gg[2], gg[2], gg[3] * gg[3])));
    const double d = wave_sum_d((double)sq);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = d;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (threadIdx.x == 0) {
      double t = 0.0;
#pragma unroll
      for (int w = 0; w < kAdamThreads / 64; ++w) t += red[w];
      part[blockIdx.x] = t;
    }
  }
}

// ---------------------------------------------------------------------------
// Sum of squares, accumulated into a device double.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(kThreads) sumsq_kernel(const T* __restrict__ x, int64_t n, double* __restrict__ acc) {
  __shared__ double red[kThreads / 64];
  float local = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float t = Elem<T>::load(x, i);
    local = fmaf(t, t, local);
  }
  double d = wave_sum_d((double)local);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = d;
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int w = 0; w < kThreads / 64; ++w) s += red[w];
    atomicAdd(acc, s);
  }
}

// Sum of the workgroup partials of adamw_vec_kernel (and the squares of the
// n % 4 tail it leaves to the scalar kernel) added to *acc, in a fixed order:
// kNormBlocks workgroups reduce contiguous ranges into part2, then one
// workgroup sums part2 and the tail.
constexpr int kNormBlocks = 256;

__global__ void __launch_bounds__(256) norm_partials_kernel(const double* __restrict__ part, int64_t nparts,
                                                            double* __restrict__ part2) {
  __shared__ double red[4];
  const int64_t per = lz_cdiv(nparts, kNormBlocks);
  const int64_t b0 = (int64_t)blockIdx.x * per, b1 = min(nparts, b0 + per);
  double t = 0.0;
  for (int64_t i = b0 + threadIdx.x; i < b1; i += 256) t += part[i];
  t = wave_sum_d(t);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = t;
  __syncthreads();
  if (threadIdx.x == 0) part2[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

template <typename G>
__global__ void __launch_bounds__(256) norm_final_kernel(const double* __restrict__ part2, const G* __restrict__ tail,
                                                         int ntail, double* __restrict__ acc) {
  __shared__ double red[4];
  double t = threadIdx.x < kNormBlocks ? part2[threadIdx.x] : 0.0;
  if (threadIdx.x < ntail) {
    const float x = Elem<G>::load(tail, threadIdx.x);
    t += (double)(x * x);
  }
  t = wave_sum_d(t);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = t;
  __syncthreads();
  if (threadIdx.x == 0) *acc += (red[0] + red[1]) + (red[2] + red[3]);
}

// Float64 words of workspace the norm-accumulating AdamW takes for n
// elements: one partial per workgroup, then kNormBlocks second-level sums.
inline int64_t adamw_norm_words(int64_t n) { return lz_cdiv(n / 4, kAdamThreads) + kNormBlocks; }

template <typename G, typename PO>
int launch_adamw(float* p, float* m, float* v, const void* g, void* pout, int64_t n, const AdamArgs& a,
                 const float* scale, const float* hyper, hipStream_t s, double* sumsq = nullptr,
                 double* ws = nullptr) {
  const G* gp = static_cast<const G*>(g);
  PO* po = static_cast<PO*>(pout);
  const bool vec = lz_aligned16(p) && lz_aligned16(m) && lz_aligned16(v) &&
                   ((reinterpret_cast<uintptr_t>(g) & (4 * sizeof(G) - 1)) == 0) &&
                   (pout == nullptr || (reinterpret_cast<uintptr_t>(pout) & (4 * sizeof(PO) - 1)) == 0);
  if (sumsq && !vec) {
    // unaligned operands take the scalar kernel: the sum of squares gets a
    // pass of its own first (the update does not change g)
    sumsq_kernel<G><<<stream_grid(n), kThreads, 0, s>>>(gp, n, sumsq);
    const int rc = lz_check_launch("lz_adamw_norm");
    if (rc) return rc;
    sumsq = nullptr;
  }
  if (vec) {
    const int64_t n4 = n / 4, tail = n - 4 * n4;
    LZ_REQUIRE(lz_cdiv(n4, kAdamThreads) < (1ll << 31), "lz_adamw: too many elements");
    const int64_t nblk = lz_cdiv(n4, kAdamThreads);
    double* part = sumsq ? ws : nullptr;
    if (n4 > 0)
      adamw_vec_kernel<G, PO><<<(unsigned)nblk, kAdamThreads, 0, s>>>(p, m, v, gp, po, n4, a, scale, hyper, part);
    if (sumsq) {
      double* part2 = ws + nblk;
      norm_partials_kernel<<<kNormBlocks, 256, 0, s>>>(ws, n4 > 0 ? nblk : 0, part2);
      norm_final_kernel<G><<<1, 256, 0, s>>>(part2, gp + 4 * n4, (int)tail, sumsq);
    }
    if (tail > 0)
      adamw_scalar_kernel<G, PO><<<1, kThreads, 0, s>>>(p + 4 * n4, m + 4 * n4, v + 4 * n4, gp + 4 * n4,
                                                        po ? po + 4 * n4 : nullptr, tail, a, scale, hyper);
  } else {
    int grid = stream_grid(n);
    adamw_scalar_kernel<G, PO><<<grid, kThreads, 0, s>>>(p, m, v, gp, po, n, a, scale, hyper);
  }
  return lz_check_launch("lz_adamw");
}

__global__ void sumsq_vec4_f32_kernel(const float* __restrict__ x, int64_t n, double* __restrict__ acc) {
  __shared__ double red[kThreads / 64];
  float local = 0.f;
  const int64_t n4 = n >> 2;
  for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < n4; q += (int64_t)gridDim.x * blockDim.x) {
    float4 t = reinterpret_cast<const float4*>(x)[q];
    local = fmaf(t.x, t.x, local);
    local = fmaf(t.y, t.y, local);
    local = fmaf(t.z, t.z, local);
    local = fmaf(t.w, t.w, local);
  }
  if (blockIdx.x == 0)
    for (int64_t i = (n4 << 2) + threadIdx.x; i < n; i += blockDim.x) local = fmaf(x[i], x[i], local);
  double d = wave_sum_d((double)local);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = d;
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int w = 0; w < kThreads / 64; ++w) s += red[w];
    atomicAdd(acc, s);
  }
}

// norm = sqrt(sum of squares) rounded to fp32 (the reference reads an fp32
// norm with .item()); scale = max/(norm + 1e-6) when clipping applies, else 1
// (zero/stage0_ddp.py:66-71).
__global__ void clip_finalize_kernel(const double* __restrict__ acc, float max_norm, float inv_grad_scale,
                                     float* __restrict__ norm_out, float* __restrict__ scale_out) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    // the gradients carry a loss scale: their norm divided by it is the true
    // norm, and the factor handed to AdamW unscales them as well as clipping
    const float norm = (float)(sqrt(*acc) * (double)inv_grad_scale);
    float scale = 1.0f;
    if (max_norm > 0.0f && norm > max_norm) scale = (float)((double)max_norm / ((double)norm + 1e-6));
    if (norm_out) *norm_out = norm;
    if (scale_out) *scale_out = scale * inv_grad_scale;
  }
}

// ---------------------------------------------------------------------------
// Fill, cast, accumulate.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void fill_kernel(T* __restrict__ x, int64_t n, T value) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) x[i] = value;
}

__global__ void fill16_kernel(uint4* __restrict__ x, int64_t n16, uint4 value) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x) x[i] = value;
}

// One 16-byte store per thread over the whole range (no loop for ranges up to
// 2^39 bytes): the launch shape that measured fastest for streaming stores.
inline int flat_grid(int64_t n16) {
  return (int)std::max<int64_t>(1, std::min<int64_t>(lz_cdiv(n16, kThreads), (int64_t)INT32_MAX));
}

template <typename S, typename D>
__global__ void cast_kernel(const S* __restrict__ src, D* __restrict__ dst, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    Elem<D>::store(dst, i, Elem<S>::load(src, i));
}

// Eight consecutive elements as floats (16-byte accesses; fp32 takes two).
template <typename T>
struct Vec8;
template <>
struct Vec8<float> {
  static __device__ __forceinline__ void load(const float* p, float (&r)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w; r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&r)[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(r[0], r[1], r[2], r[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(r[4], r[5], r[6], r[7]);
  }
};
template <>
struct Vec8<uint16_t> {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {  // round to nearest even
    const f32x2_t f = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
  }
  static __device__ __forceinline__ void load(const uint16_t* p, float (&r)[8]) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      r[2 * k] = __uint_as_float(w[k] << 16);
      r[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ void store(uint16_t* p, const float (&r)[8]) {
    *reinterpret_cast<uint4*>(p) = make_uint4(pack(r[0], r[1]), pack(r[2], r[3]), pack(r[4], r[5]), pack(r[6], r[7]));
  }
};
template <>
struct Vec8<_Float16> {
  static __device__ __forceinline__ void load(const _Float16* p, float (&r)[8]) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      r[2 * k] = h2f(w[k] & 0xffff);
      r[2 * k + 1] = h2f(w[k] >> 16);
    }
  }
  static __device__ __forceinline__ void store(_Float16* p, const float (&r)[8]) {
    *reinterpret_cast<uint4*>(p) =
        make_uint4(pack_f16x2(r[0], r[1]), pack_f16x2(r[2], r[3]), pack_f16x2(r[4], r[5]), pack_f16x2(r[6], r[7]));
  }
};

// Vector paths: one 8-element group per thread over a full grid.
template <typename S, typename D>
__global__ void __launch_bounds__(kThreads) cast_vec8_kernel(const S* __restrict__ src, D* __restrict__ dst, int64_t n8) {
  const int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (q >= n8) return;
  float r[8];
  Vec8<S>::load(src + 8 * q, r);
  Vec8<D>::store(dst + 8 * q, r);
}

template <typename S>
__global__ void __launch_bounds__(kThreads) axpy_vec8_kernel(float* __restrict__ dst, const S* __restrict__ src,
                                                             int64_t n8, float alpha, int unit_alpha) {
  const int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (q >= n8) return;
  float a[8], d[8];
  Vec8<S>::load(src + 8 * q, a);
  Vec8<float>::load(dst + 8 * q, d);
#pragma unroll
  for (int e = 0; e < 8; ++e) d[e] = unit_alpha ? d[e] + a[e] : fmaf(alpha, a[e], d[e]);
  Vec8<float>::store(dst + 8 * q, d);
}

inline unsigned vec_grid(int64_t n8) { return (unsigned)std::max<int64_t>(1, lz_cdiv(n8, kThreads)); }

// dst(f32) += alpha * src
template <typename S>
__global__ void axpy_f32_kernel(float* __restrict__ dst, const S* __restrict__ src, int64_t n, float alpha, int unit_alpha) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float s = Elem<S>::load(src, i);
    dst[i] = unit_alpha ? dst[i] + s : fmaf(alpha, s, dst[i]);
  }
}

// dst = round_T(dst + src), both in the storage type T (torch's in-place add).
template <typename T>
__global__ void add_inplace_kernel(T* __restrict__ dst, const T* __restrict__ src, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    Elem<T>::store(dst, i, Elem<T>::load(dst, i) + Elem<T>::load(src, i));
}

// x *= alpha (in the storage type).
template <typename T>
__global__ void scale_kernel(T* __restrict__ x, int64_t n, float alpha) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    Elem<T>::store(x, i, Elem<T>::load(x, i) * alpha);
}

// x *= *scale (a device scalar, e.g. an upstream loss gradient).
template <typename T>
__global__ void scale_dev_kernel(T* __restrict__ x, int64_t n, const float* __restrict__ scale) {
  const float a = *scale;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    Elem<T>::store(x, i, Elem<T>::load(x, i) * a);
}

// ---------------------------------------------------------------------------
// Multi-tensor gather/scatter.  `table` is a device int64 array of nseg
// records {ptr, numel, flat_offset}, sorted by flat_offset.  A record with a
// null ptr reads as zeros (a parameter without a gradient).
// ---------------------------------------------------------------------------
constexpr int64_t kChunk = 8192;

__device__ __forceinline__ int find_segment(const int64_t* table, int nseg, int64_t pos) {
  // first segment whose end is > pos
  int lo = 0, hi = nseg;
  while (lo < hi) {
    int mid = (lo + hi) >> 1;
    if (table[3 * mid + 2] + table[3 * mid + 1] <= pos) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// mode 0: dst = src ; mode 1: dst(f32) += src
template <typename S, typename D>
__global__ void __launch_bounds__(kThreads) mt_gather_kernel(const int64_t* __restrict__ table, int nseg, D* __restrict__ dst,
                                                              int64_t begin, int64_t end, int mode) {
  const int64_t nchunks = lz_cdiv(end - begin, kChunk);
  for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const int64_t c0 = begin + c * kChunk;
    const int64_t c1 = min(c0 + kChunk, end);
    for (int s = find_segment(table, nseg, c0); s < nseg; ++s) {
      const S* ptr = reinterpret_cast<const S*>(table[3 * s]);
      const int64_t numel = table[3 * s + 1], off = table[3 * s + 2];
      if (off >= c1) break;
      const int64_t lo = max(c0, off), hi = min(c1, off + numel);
      for (int64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) {
        float val = ptr ? Elem<S>::load(ptr, i - off) : 0.0f;
        if (mode == 1) {
          float* d = reinterpret_cast<float*>(dst);
          d[i - begin] += val;
        } else {
          Elem<D>::store(dst, i - begin, val);
        }
      }
    }
  }
}

template <typename S, typename D>
__global__ void __launch_bounds__(kThreads) mt_scatter_kernel(const S* __restrict__ src, const int64_t* __restrict__ table,
                                                               int nseg, int64_t begin, int64_t end) {
  const int64_t nchunks = lz_cdiv(end - begin, kChunk);
  for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const int64_t c0 = begin + c * kChunk;
    const int64_t c1 = min(c0 + kChunk, end);
    for (int s = find_segment(table, nseg, c0); s < nseg; ++s) {
      D* ptr = reinterpret_cast<D*>(table[3 * s]);
      const int64_t numel = table[3 * s + 1], off = table[3 * s + 2];
      if (off >= c1) break;
      if (!ptr) continue;
      const int64_t lo = max(c0, off), hi = min(c1, off + numel);
      for (int64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) Elem<D>::store(ptr, i - off, Elem<S>::load(src, i - begin));
    }
  }
}

// Segment table passed by value in the kernel arguments (no device copy of
// the table, so a host-built table costs no host<->device synchronisation).
constexpr int kArgSegs = 48;
struct SegArgs {
  int64_t ptr[kArgSegs];
  int64_t numel[kArgSegs];
  int64_t off[kArgSegs];
  int n;
};

__device__ __forceinline__ int find_segment_args(const SegArgs& t, int64_t pos) {
  int lo = 0, hi = t.n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (t.off[mid] + t.numel[mid] <= pos) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

template <typename S, typename D>
__global__ void __launch_bounds__(kThreads) mt_gather_args_kernel(const SegArgs t, D* __restrict__ dst, int64_t begin,
                                                                   int64_t end, int64_t dst_base, int mode) {
  const int64_t nchunks = lz_cdiv(end - begin, kChunk);
  for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const int64_t c0 = begin + c * kChunk;
    const int64_t c1 = min(c0 + kChunk, end);
    for (int s = find_segment_args(t, c0); s < t.n; ++s) {
      const S* ptr = reinterpret_cast<const S*>(t.ptr[s]);
      const int64_t numel = t.numel[s], off = t.off[s];
      if (off >= c1) break;
      const int64_t lo = max(c0, off), hi = min(c1, off + numel);
      int64_t i0 = lo;
      // 8 elements per thread where source and destination are 16-byte aligned
      // at the same element
      if (ptr && ((lo - off) & 7) == 0 && ((lo - dst_base) & 7) == 0 &&
          ((reinterpret_cast<uintptr_t>(ptr) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0) {
        const int64_t nv = (hi - lo) >> 3;
        const S* sp = ptr + (lo - off);
        const int64_t dofs = lo - dst_base;
        const int64_t bd = blockDim.x;
        int64_t v = threadIdx.x;
        // four groups per thread at a time, their loads issued together (one
        // group per round trip left too few bytes in flight to reach the
        // copy rate)
        for (; v + 3 * bd < nv; v += 4 * bd) {
          float r[4][8];
#pragma unroll
          for (int u = 0; u < 4; ++u) Vec8<S>::load(sp + 8 * (v + u * bd), r[u]);
          if (mode == 1) {
            float* dp = reinterpret_cast<float*>(dst) + dofs;
            float d[4][8];
#pragma unroll
            for (int u = 0; u < 4; ++u) Vec8<float>::load(dp + 8 * (v + u * bd), d[u]);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
#pragma unroll
              for (int e = 0; e < 8; ++e) d[u][e] += r[u][e];
              Vec8<float>::store(dp + 8 * (v + u * bd), d[u]);
            }
          } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) Vec8<D>::store(dst + dofs + 8 * (v + u * bd), r[u]);
          }
        }
        for (; v < nv; v += bd) {
          float r[8];
          Vec8<S>::load(sp + 8 * v, r);
          if (mode == 1) {
            float d[8];
            float* dp = reinterpret_cast<float*>(dst) + dofs + 8 * v;
            Vec8<float>::load(dp, d);
#pragma unroll
            for (int e = 0; e < 8; ++e) d[e] += r[e];
            Vec8<float>::store(dp, d);
          } else {
            Vec8<D>::store(dst + dofs + 8 * v, r);
          }
        }
        i0 = lo + 8 * nv;
      }
      for (int64_t i = i0 + threadIdx.x; i < hi; i += blockDim.x) {
        const float val = ptr ? Elem<S>::load(ptr, i - off) : 0.0f;
        if (mode == 1) reinterpret_cast<float*>(dst)[i - dst_base] += val;
        else Elem<D>::store(dst, i - dst_base, val);
      }
    }
  }
}

template <typename S, typename D>
__global__ void __launch_bounds__(kThreads) mt_scatter_args_kernel(const S* __restrict__ src, const SegArgs t, int64_t begin,
                                                                    int64_t end, int64_t src_base) {
  const int64_t nchunks = lz_cdiv(end - begin, kChunk);
  for (int64_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
    const int64_t c0 = begin + c * kChunk;
    const int64_t c1 = min(c0 + kChunk, end);
    for (int s = find_segment_args(t, c0); s < t.n; ++s) {
      D* ptr = reinterpret_cast<D*>(t.ptr[s]);
      const int64_t numel = t.numel[s], off = t.off[s];
      if (off >= c1) break;
      if (!ptr) continue;
      const int64_t lo = max(c0, off), hi = min(c1, off + numel);
      for (int64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) Elem<D>::store(ptr, i - off, Elem<S>::load(src, i - src_base));
    }
  }
}

// Splits a host table into launches of at most kArgSegs segments, each over
// the part of [begin, end) its segments cover.  kind 0 = gather, 1 = scatter.
template <typename S, typename D>
int run_host_table(int kind, const int64_t* host, int nseg, void* flat, int64_t begin, int64_t end, int accumulate,
                   hipStream_t st) {
  for (int s0 = 0; s0 < nseg; s0 += kArgSegs) {
    SegArgs a;
    a.n = std::min(kArgSegs, nseg - s0);
    for (int j = 0; j < a.n; ++j) {
      a.ptr[j] = host[3 * (s0 + j)];
      a.numel[j] = host[3 * (s0 + j) + 1];
      a.off[j] = host[3 * (s0 + j) + 2];
    }
    const int64_t lo = std::max(begin, a.off[0]);
    const int64_t hi = std::min(end, a.off[a.n - 1] + a.numel[a.n - 1]);
    if (hi <= lo) continue;
    const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(lz_cdiv(hi - lo, kChunk), (int64_t)lz_num_cus() * 8));
    if (kind == 0)
      mt_gather_args_kernel<S, D><<<grid, kThreads, 0, st>>>(a, static_cast<D*>(flat), lo, hi, begin, accumulate);
    else
      mt_scatter_args_kernel<S, D><<<grid, kThreads, 0, st>>>(static_cast<const S*>(flat), a, lo, hi, begin);
    int rc = lz_check_launch(kind == 0 ? "lz_mt_gather_host" : "lz_mt_scatter_host");
    if (rc) return rc;
  }
  return LZ_OK;
}

int check_host_table(const int64_t* host, int nseg) {
  LZ_REQUIRE(host && nseg > 0, "multi-tensor: empty table");
  for (int i = 0; i < nseg; ++i) {
    LZ_REQUIRE(host[3 * i + 1] >= 0, "multi-tensor: negative segment size");
    if (i > 0) LZ_REQUIRE(host[3 * i + 2] >= host[3 * (i - 1) + 2] + host[3 * (i - 1) + 1], "multi-tensor: segments overlap or are unsorted");
  }
  return LZ_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Multi-tensor AdamW and sum of squares: one launch over up to kMultiSegs
// tensors, whose pointers travel by value in the kernel arguments.  Every
// workgroup takes one chunk of kMultiChunk elements of one tensor (chunks are
// numbered tensor after tensor; chunk0 holds each tensor's first chunk), so
// the element math is exactly that of the one-tensor kernels.
// ---------------------------------------------------------------------------
constexpr int kMultiSegs = 24;
constexpr int64_t kMultiChunk = 4096;

struct MultiSegs {
  int64_t p[kMultiSegs], m[kMultiSegs], v[kMultiSegs], g[kMultiSegs], po[kMultiSegs];
  int64_t numel[kMultiSegs];
  int64_t chunk0[kMultiSegs + 1];
  int n;
};

// the tensor whose chunk range holds chunk c (the last with chunk0 <= c)
__device__ __forceinline__ int multi_segment(const int64_t* chunk0, int n, int64_t c) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (chunk0[mid] <= c) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

template <typename G, typename PO>
__global__ void __launch_bounds__(kThreads) adamw_multi_kernel(const MultiSegs t, AdamArgs a0,
                                                               const float* __restrict__ scale_ptr,
                                                               const float* __restrict__ hyper) {
  const AdamArgs a = with_hyper(a0, hyper);
  const float scale = scale_ptr ? *scale_ptr : 1.0f;
  const int64_t c = blockIdx.x;
  const int sg = multi_segment(t.chunk0, t.n, c);
  const int64_t i0 = (c - t.chunk0[sg]) * kMultiChunk, i1 = min(i0 + kMultiChunk, t.numel[sg]);
  float* p = reinterpret_cast<float*>(t.p[sg]);
  float* m = reinterpret_cast<float*>(t.m[sg]);
  float* v = reinterpret_cast<float*>(t.v[sg]);
  const G* g = reinterpret_cast<const G*>(t.g[sg]);
  PO* po = reinterpret_cast<PO*>(t.po[sg]);
  // Four elements per thread and access when every array of this tensor is
  // aligned to four of its elements (chunk starts are multiples of
  // kMultiChunk, so alignment depends only on the base pointers); the same
  // arithmetic per element as the scalar loop, so the same bits.
  const bool vec = ((t.p[sg] | t.m[sg] | t.v[sg]) & 15) == 0 && (t.g[sg] & (4 * sizeof(G) - 1)) == 0 &&
                   (t.po[sg] & (4 * sizeof(PO) - 1)) == 0;
  int64_t tail = i0;
  if (vec) {
    const int64_t n4 = (i1 - i0) >> 2;
    for (int64_t q = threadIdx.x; q < n4; q += blockDim.x) {
      const int64_t i = i0 + 4 * q;
      float4 pv = *reinterpret_cast<const float4*>(p + i);
      float4 mv = *reinterpret_cast<const float4*>(m + i);
      float4 vv = *reinterpret_cast<const float4*>(v + i);
      float gv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) gv[e] = Elem<G>::load(g, i + e);
      float* pe = &pv.x;
      float* me = &mv.x;
      float* ve = &vv.x;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float gg = scale_ptr ? gv[e] * scale : gv[e];
        adam_elem(pe[e], me[e], ve[e], gg, a);
      }
      *reinterpret_cast<float4*>(p + i) = pv;
      *reinterpret_cast<float4*>(m + i) = mv;
      *reinterpret_cast<float4*>(v + i) = vv;
      if (po)
#pragma unroll
        for (int e = 0; e < 4; ++e) Elem<PO>::store(po, i + e, pe[e]);
    }
    tail = i0 + 4 * n4;
  }
  for (int64_t i = tail + threadIdx.x; i < i1; i += blockDim.x) {
    float pp = p[i], mm = m[i], vv = v[i];
    float gg = Elem<G>::load(g, i);
    if (scale_ptr) gg = gg * scale;
    adam_elem(pp, mm, vv, gg, a);
    p[i] = pp;
    m[i] = mm;
    v[i] = vv;
    if (po) Elem<PO>::store(po, i, pp);
  }
}

template <typename T>
__global__ void __launch_bounds__(kThreads) sumsq_multi_kernel(const MultiSegs t, double* __restrict__ acc) {
  __shared__ double red[kThreads / 64];
  const int64_t c = blockIdx.x;
  const int sg = multi_segment(t.chunk0, t.n, c);
  const int64_t i0 = (c - t.chunk0[sg]) * kMultiChunk, i1 = min(i0 + kMultiChunk, t.numel[sg]);
  const T* x = reinterpret_cast<const T*>(t.g[sg]);
  float local = 0.f;
  for (int64_t i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
    const float e = Elem<T>::load(x, i);
    local = fmaf(e, e, local);
  }
  double d = wave_sum_d((double)local);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = d;
  __syncthreads();
  if (threadIdx.x == 0) {
    double sum = 0.0;
    for (int w = 0; w < kThreads / 64; ++w) sum += red[w];
    atomicAdd(acc, sum);
  }
}

// Calls f with a value of the storage type of `dtype` (float, uint16_t for
// bf16, _Float16 for fp16).
template <typename Fn>
int with_elem(int dtype, Fn&& f) {
  if (dtype == LZ_F32) return f(float{});
  if (dtype == LZ_BF16) return f(uint16_t{});
  return f(_Float16{});
}

template <typename S, typename D>
int cast_typed(const void* src, void* dst, int64_t n, hipStream_t s) {
  if (lz_aligned16(src) && lz_aligned16(dst) && n >= 8) {
    const int64_t n8 = n / 8, done = 8 * n8;
    cast_vec8_kernel<S, D><<<vec_grid(n8), kThreads, 0, s>>>((const S*)src, (D*)dst, n8);
    int rc = lz_check_launch("lz_cast");
    if (rc || done == n) return rc;
    return cast_typed<S, D>(static_cast<const S*>(src) + done, static_cast<D*>(dst) + done, n - done, s);
  }
  cast_kernel<S, D><<<stream_grid(n), kThreads, 0, s>>>((const S*)src, (D*)dst, n);
  return lz_check_launch("lz_cast");
}

// ===========================================================================
// Exported entry points.
// ===========================================================================

// Fused AdamW over n elements of an fp32 master (p), moments (m, v) and a
// gradient (g, fp32 or bf16), optionally scaled by *grad_scale (the clip factor,
// read on the device) and optionally writing the updated parameter in a low
// precision copy (p_out).  Hyper-parameters arrive as doubles, like the
// reference's Python floats; bias corrections use `step` (1-based).
namespace {

int adamw_entry(float* p, float* m, float* v, const void* g, int g_dtype, void* p_out, int p_out_dtype, int64_t n,
                double lr, double beta1, double beta2, double eps, double weight_decay, int64_t step,
                const float* grad_scale, const float* hyper, void* stream, double* sumsq = nullptr,
                double* ws = nullptr) {
  if (n == 0) return LZ_OK;
  LZ_REQUIRE(p && m && v && g && n > 0, "lz_adamw: bad arguments");
  const double bc1 = 1.0 - pow(beta1, (double)step);
  const double bc2 = 1.0 - pow(beta2, (double)step);
  AdamArgs a;
  a.beta1 = (float)beta1;
  a.beta2 = (float)beta2;
  a.omb1 = (float)(1.0 - beta1);
  a.omb2 = (float)(1.0 - beta2);
  a.wd_factor = (float)(1.0 - lr * weight_decay);
  a.apply_wd = weight_decay != 0.0;
  a.sqrt_bc2 = (float)sqrt(bc2);
  a.eps = (float)eps;
  a.neg_step = (float)(-(lr / bc1));
  hipStream_t s = lz_stream(stream);
  const bool gb = g_dtype == LZ_BF16, gh = g_dtype == LZ_F16;
  LZ_REQUIRE(g_dtype == LZ_BF16 || g_dtype == LZ_F32 || g_dtype == LZ_F16, "lz_adamw: bad grad dtype %d", g_dtype);
  if (gh) {  // fp16 models: fp16 gradients, fp16 (or no) parameter copy
    if (p_out == nullptr || p_out_dtype == LZ_F32)
      return launch_adamw<_Float16, float>(p, m, v, g, p_out, n, a, grad_scale, hyper, s, sumsq, ws);
    LZ_REQUIRE(p_out_dtype == LZ_F16, "lz_adamw: bad output dtype %d for fp16 gradients", p_out_dtype);
    return launch_adamw<_Float16, _Float16>(p, m, v, g, p_out, n, a, grad_scale, hyper, s, sumsq, ws);
  }
  if (p_out == nullptr || p_out_dtype == LZ_F32) {
    return gb ? launch_adamw<uint16_t, float>(p, m, v, g, p_out, n, a, grad_scale, hyper, s, sumsq, ws)
              : launch_adamw<float, float>(p, m, v, g, p_out, n, a, grad_scale, hyper, s, sumsq, ws);
  }
  LZ_REQUIRE(p_out_dtype == LZ_BF16, "lz_adamw: bad output dtype %d", p_out_dtype);
  return gb ? launch_adamw<uint16_t, uint16_t>(p, m, v, g, p_out, n, a, grad_scale, hyper, s, sumsq, ws)
            : launch_adamw<float, uint16_t>(p, m, v, g, p_out, n, a, grad_scale, hyper, s, sumsq, ws);
}

// One thread: advances the device step counter and writes the factors that
// depend on it, in the same double arithmetic as the host path of lz_adamw.
__global__ void adamw_step_kernel(int64_t* __restrict__ step, double lr, double beta1, double beta2,
                                  double weight_decay, float* __restrict__ hyper) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  const int64_t t = *step + 1;
  *step = t;
  const double bc1 = 1.0 - pow(beta1, (double)t);
  const double bc2 = 1.0 - pow(beta2, (double)t);
  hyper[0] = (float)(-(lr / bc1));
  hyper[1] = (float)sqrt(bc2);
  hyper[2] = (float)(1.0 - lr * weight_decay);
}

}  // namespace

LZ_EXPORT int lz_adamw(float* p, float* m, float* v, const void* g, int g_dtype, void* p_out, int p_out_dtype,
                            int64_t n, double lr, double beta1, double beta2, double eps, double weight_decay,
                            int64_t step, const float* grad_scale, void* stream) {
  LZ_REQUIRE(step >= 1, "lz_adamw: step must be >= 1");
  return adamw_entry(p, m, v, g, g_dtype, p_out, p_out_dtype, n, lr, beta1, beta2, eps, weight_decay, step, grad_scale,
                     nullptr, stream);
}

LZ_EXPORT int64_t lz_adamw_norm_workspace(int64_t n) { return n > 0 ? adamw_norm_words(n) : 0; }

LZ_EXPORT int lz_adamw_norm(float* p, float* m, float* v, const void* g, int g_dtype, void* p_out, int p_out_dtype,
                            int64_t n, double lr, double beta1, double beta2, double eps, double weight_decay,
                            int64_t step, const float* grad_scale, double* acc, double* workspace,
                            int64_t workspace_words, void* stream) {
  LZ_REQUIRE(step >= 1, "lz_adamw_norm: step must be >= 1");
  LZ_REQUIRE(acc, "lz_adamw_norm: null accumulator");
  LZ_REQUIRE(n >= 0, "lz_adamw_norm: bad element count");
  LZ_REQUIRE(workspace && workspace_words >= lz_adamw_norm_workspace(n),
             "lz_adamw_norm: workspace of %lld float64 words, %lld needed", (long long)workspace_words,
             (long long)lz_adamw_norm_workspace(n));
  return adamw_entry(p, m, v, g, g_dtype, p_out, p_out_dtype, n, lr, beta1, beta2, eps, weight_decay, step, grad_scale,
                     nullptr, stream, acc, workspace);
}

LZ_EXPORT int lz_adamw_step(int64_t* step, double lr, double beta1, double beta2, double weight_decay, float* hyper,
                            void* stream) {
  LZ_REQUIRE(step && hyper, "lz_adamw_step: null pointer");
  adamw_step_kernel<<<1, 64, 0, lz_stream(stream)>>>(step, lr, beta1, beta2, weight_decay, hyper);
  return lz_check_launch("lz_adamw_step");
}

LZ_EXPORT int lz_adamw_dev(float* p, float* m, float* v, const void* g, int g_dtype, void* p_out, int p_out_dtype,
                           int64_t n, double beta1, double beta2, double eps, double weight_decay, const float* hyper,
                           const float* grad_scale, void* stream) {
  LZ_REQUIRE(hyper, "lz_adamw_dev: null step factors");
  // lr and the step come from `hyper`; the host factors are placeholders
  return adamw_entry(p, m, v, g, g_dtype, p_out, p_out_dtype, n, 0.0, beta1, beta2, eps, weight_decay, 1, grad_scale,
                     hyper, stream);
}

LZ_EXPORT int lz_sumsq(const void* x, int dtype, int64_t n, double* acc, void* stream) {
  LZ_REQUIRE(n >= 0 && acc, "lz_sumsq: bad arguments");
  if (n == 0) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  if (dtype == LZ_F32) {
    if (lz_aligned16(x)) sumsq_vec4_f32_kernel<<<stream_grid(n / 4 + 1), kThreads, 0, s>>>((const float*)x, n, acc);
    else sumsq_kernel<float><<<stream_grid(n), kThreads, 0, s>>>((const float*)x, n, acc);
  } else if (dtype == LZ_BF16) {
    sumsq_kernel<uint16_t><<<stream_grid(n), kThreads, 0, s>>>((const uint16_t*)x, n, acc);
  } else if (dtype == LZ_F16) {
    sumsq_kernel<_Float16><<<stream_grid(n), kThreads, 0, s>>>((const _Float16*)x, n, acc);
  } else {
    return lz_set_error(LZ_EINVAL, "lz_sumsq: bad dtype %d", dtype);
  }
  return lz_check_launch("lz_sumsq");
}

namespace {

// Fills `t` with rows [r0, r1) of a host table of `cols` int64 columns (the
// tensor pointer columns given by `ptr_cols`, numel last), skipping empty
// tensors; returns the number of chunks.
int64_t fill_multi(MultiSegs& t, const int64_t* table, int cols, int r0, int r1) {
  t = MultiSegs{};
  int64_t chunks = 0;
  for (int r = r0; r < r1; ++r) {
    const int64_t* row = table + (int64_t)r * cols;
    const int64_t n = row[cols - 1];
    if (n <= 0) continue;
    const int k = t.n++;
    if (cols == 6) {
      t.p[k] = row[0];
      t.m[k] = row[1];
      t.v[k] = row[2];
      t.g[k] = row[3];
      t.po[k] = row[4];
    } else {
      t.g[k] = row[0];
    }
    t.numel[k] = n;
    t.chunk0[k] = chunks;
    chunks += lz_cdiv(n, kMultiChunk);
  }
  t.chunk0[t.n] = chunks;
  return chunks;
}

}  // namespace

// AdamW over nseg tensors in one launch per 24 tensors: table holds nseg rows
// {p (fp32 master), m, v, g, p_out (0 = none), numel}; every row shares
// g_dtype and p_out_dtype.  The same update as lz_adamw on each tensor, bit
// for bit.  With hyper set (written by lz_adamw_step) lr and step are unused.
LZ_EXPORT int lz_adamw_multi(const int64_t* table, int nseg, int g_dtype, int p_out_dtype, double lr, double beta1,
                             double beta2, double eps, double weight_decay, int64_t step, const float* hyper,
                             const float* grad_scale, void* stream) {
  LZ_REQUIRE(table && nseg >= 0, "lz_adamw_multi: bad table");
  LZ_REQUIRE(hyper || step >= 1, "lz_adamw_multi: step must be >= 1");
  LZ_REQUIRE(g_dtype == LZ_BF16 || g_dtype == LZ_F32 || g_dtype == LZ_F16, "lz_adamw_multi: bad grad dtype %d",
             g_dtype);
  LZ_REQUIRE(p_out_dtype == LZ_BF16 || p_out_dtype == LZ_F32 || p_out_dtype == LZ_F16,
             "lz_adamw_multi: bad output dtype %d", p_out_dtype);
  LZ_REQUIRE((g_dtype == LZ_F16) == (p_out_dtype == LZ_F16) || p_out_dtype == LZ_F32,
             "lz_adamw_multi: fp16 gradients go with fp16 (or fp32) parameters (%d, %d)", g_dtype, p_out_dtype);
  for (int r = 0; r < nseg; ++r) {
    const int64_t* row = table + (int64_t)r * 6;
    LZ_REQUIRE(row[5] >= 0, "lz_adamw_multi: negative size in row %d", r);
    LZ_REQUIRE(row[5] == 0 || (row[0] && row[1] && row[2] && row[3]), "lz_adamw_multi: null pointer in row %d", r);
  }
  const double bc1 = 1.0 - pow(beta1, (double)(hyper ? 1 : step));
  const double bc2 = 1.0 - pow(beta2, (double)(hyper ? 1 : step));
  AdamArgs a;
  a.beta1 = (float)beta1;
  a.beta2 = (float)beta2;
  a.omb1 = (float)(1.0 - beta1);
  a.omb2 = (float)(1.0 - beta2);
  a.wd_factor = (float)(1.0 - lr * weight_decay);
  a.apply_wd = weight_decay != 0.0;
  a.sqrt_bc2 = (float)sqrt(bc2);
  a.eps = (float)eps;
  a.neg_step = (float)(-(lr / bc1));
  hipStream_t s = lz_stream(stream);
  const bool gb = g_dtype == LZ_BF16, ob = p_out_dtype == LZ_BF16, gh = g_dtype == LZ_F16, oh = p_out_dtype == LZ_F16;
  for (int r0 = 0; r0 < nseg; r0 += kMultiSegs) {
    MultiSegs t;
    const int64_t chunks = fill_multi(t, table, 6, r0, min(nseg, r0 + kMultiSegs));
    if (chunks == 0) continue;
    LZ_REQUIRE(chunks < (1ll << 31), "lz_adamw_multi: too many chunks");
    const unsigned grid = (unsigned)chunks;
    if (gh && oh) adamw_multi_kernel<_Float16, _Float16><<<grid, kThreads, 0, s>>>(t, a, grad_scale, hyper);
    else if (gh) adamw_multi_kernel<_Float16, float><<<grid, kThreads, 0, s>>>(t, a, grad_scale, hyper);
    else if (gb && ob) adamw_multi_kernel<uint16_t, uint16_t><<<grid, kThreads, 0, s>>>(t, a, grad_scale, hyper);
    else if (gb) adamw_multi_kernel<uint16_t, float><<<grid, kThreads, 0, s>>>(t, a, grad_scale, hyper);
    else if (ob) adamw_multi_kernel<float, uint16_t><<<grid, kThreads, 0, s>>>(t, a, grad_scale, hyper);
    else adamw_multi_kernel<float, float><<<grid, kThreads, 0, s>>>(t, a, grad_scale, hyper);
    int rc = lz_check_launch("lz_adamw_multi");
    if (rc) return rc;
  }
  return LZ_OK;
}

// *acc += sum of squares over nseg tensors of one dtype (table rows {x, numel}),
// one launch per 24 tensors.
LZ_EXPORT int lz_sumsq_multi(const int64_t* table, int nseg, int dtype, double* acc, void* stream) {
  LZ_REQUIRE(table && nseg >= 0 && acc, "lz_sumsq_multi: bad arguments");
  LZ_REQUIRE(dtype == LZ_BF16 || dtype == LZ_F32 || dtype == LZ_F16, "lz_sumsq_multi: bad dtype %d", dtype);
  for (int r = 0; r < nseg; ++r)
    LZ_REQUIRE(table[2 * r + 1] >= 0 && (table[2 * r + 1] == 0 || table[2 * r]), "lz_sumsq_multi: bad row %d", r);
  hipStream_t s = lz_stream(stream);
  for (int r0 = 0; r0 < nseg; r0 += kMultiSegs) {
    MultiSegs t;
    const int64_t chunks = fill_multi(t, table, 2, r0, min(nseg, r0 + kMultiSegs));
    if (chunks == 0) continue;
    LZ_REQUIRE(chunks < (1ll << 31), "lz_sumsq_multi: too many chunks");
    if (dtype == LZ_BF16) sumsq_multi_kernel<uint16_t><<<(unsigned)chunks, kThreads, 0, s>>>(t, acc);
    else if (dtype == LZ_F16) sumsq_multi_kernel<_Float16><<<(unsigned)chunks, kThreads, 0, s>>>(t, acc);
    else sumsq_multi_kernel<float><<<(unsigned)chunks, kThreads, 0, s>>>(t, acc);
    int rc = lz_check_launch("lz_sumsq_multi");
    if (rc) return rc;
  }
  return LZ_OK;
}

LZ_EXPORT int lz_clip_finalize(const double* acc, float max_norm, float inv_grad_scale, float* norm_out,
                               float* scale_out, void* stream) {
  LZ_REQUIRE(acc, "lz_clip_finalize: null accumulator");
  LZ_REQUIRE(inv_grad_scale > 0.f, "lz_clip_finalize: inverse loss scale must be positive");
  clip_finalize_kernel<<<1, 64, 0, lz_stream(stream)>>>(acc, max_norm, inv_grad_scale, norm_out, scale_out);
  return lz_check_launch("lz_clip_finalize");
}

LZ_EXPORT int lz_fill(void* x, int dtype, int64_t n, double value, void* stream) {
  LZ_REQUIRE(n >= 0, "lz_fill: negative n");
  if (n == 0) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  if (dtype == LZ_F32) {
    const float f = (float)value;
    if (lz_aligned16(x) && n % 4 == 0) {
      uint32_t u = __builtin_bit_cast(uint32_t, f);
      fill16_kernel<<<flat_grid(n / 4), kThreads, 0, s>>>((uint4*)x, n / 4, make_uint4(u, u, u, u));
    } else {
      fill_kernel<float><<<stream_grid(n), kThreads, 0, s>>>((float*)x, n, f);
    }
  } else if (dtype == LZ_BF16) {
    // host-side RNE rounding of the fill value
    uint32_t u = __builtin_bit_cast(uint32_t, (float)value);
    uint16_t h = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    if (lz_aligned16(x) && n % 8 == 0) {
      uint32_t w = (uint32_t)h | ((uint32_t)h << 16);
      fill16_kernel<<<flat_grid(n / 8), kThreads, 0, s>>>((uint4*)x, n / 8, make_uint4(w, w, w, w));
    } else {
      fill_kernel<uint16_t><<<stream_grid(n), kThreads, 0, s>>>((uint16_t*)x, n, h);
    }
  } else if (dtype == LZ_F16) {
    const _Float16 h = (_Float16)value;  // host conversion, round to nearest even
    const uint16_t hb = __builtin_bit_cast(uint16_t, h);
    if (lz_aligned16(x) && n % 8 == 0) {
      const uint32_t w = (uint32_t)hb | ((uint32_t)hb << 16);
      fill16_kernel<<<flat_grid(n / 8), kThreads, 0, s>>>((uint4*)x, n / 8, make_uint4(w, w, w, w));
    } else {
      fill_kernel<uint16_t><<<stream_grid(n), kThreads, 0, s>>>((uint16_t*)x, n, hb);
    }
  } else if (dtype == kFillF64) {  // float64 (accumulators)
    fill_kernel<double><<<stream_grid(n), kThreads, 0, s>>>((double*)x, n, value);
  } else {
    return lz_set_error(LZ_EINVAL, "lz_fill: bad dtype %d", dtype);
  }
  return lz_check_launch("lz_fill");
}

LZ_EXPORT int lz_cast(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n, void* stream) {
  LZ_REQUIRE(n >= 0, "lz_cast: negative n");
  LZ_REQUIRE(src_dtype >= LZ_F32 && src_dtype <= LZ_F16 && dst_dtype >= LZ_F32 && dst_dtype <= LZ_F16,
             "lz_cast: bad dtypes %d->%d", src_dtype, dst_dtype);
  if (n == 0) return LZ_OK;
  return with_elem(src_dtype, [&](auto s0) {
    using S = decltype(s0);
    return with_elem(dst_dtype, [&](auto d0) {
      using D = decltype(d0);
      return cast_typed<S, D>(src, dst, n, lz_stream(stream));
    });
  });
}

LZ_EXPORT int lz_axpy_f32(float* dst, const void* src, int src_dtype, int64_t n, float alpha, void* stream) {
  LZ_REQUIRE(n >= 0 && dst, "lz_axpy_f32: bad arguments");
  if (n == 0) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  const int unit = alpha == 1.0f;
  if ((src_dtype == LZ_BF16 || src_dtype == LZ_F32) && lz_aligned16(dst) && lz_aligned16(src) && n >= 8) {
    const int64_t n8 = n / 8, done = 8 * n8;
    if (src_dtype == LZ_BF16) axpy_vec8_kernel<uint16_t><<<vec_grid(n8), kThreads, 0, s>>>(dst, (const uint16_t*)src, n8, alpha, unit);
    else axpy_vec8_kernel<float><<<vec_grid(n8), kThreads, 0, s>>>(dst, (const float*)src, n8, alpha, unit);
    int rc = lz_check_launch("lz_axpy_f32");
    if (rc || done == n) return rc;
    return lz_axpy_f32(dst + done, static_cast<const char*>(src) + done * (src_dtype == LZ_F32 ? 4 : 2), src_dtype,
                       n - done, alpha, stream);
  }
  if (src_dtype == LZ_BF16) axpy_f32_kernel<uint16_t><<<stream_grid(n), kThreads, 0, s>>>(dst, (const uint16_t*)src, n, alpha, unit);
  else if (src_dtype == LZ_F16) axpy_f32_kernel<_Float16><<<stream_grid(n), kThreads, 0, s>>>(dst, (const _Float16*)src, n, alpha, unit);
  else if (src_dtype == LZ_F32) axpy_f32_kernel<float><<<stream_grid(n), kThreads, 0, s>>>(dst, (const float*)src, n, alpha, unit);
  else return lz_set_error(LZ_EINVAL, "lz_axpy_f32: bad dtype %d", src_dtype);
  return lz_check_launch("lz_axpy_f32");
}

LZ_EXPORT int lz_scale_dev(void* x, int dtype, int64_t n, const float* scale, void* stream) {
  LZ_REQUIRE(n >= 0 && scale, "lz_scale_dev: bad arguments");
  if (n == 0) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  if (dtype == LZ_BF16) scale_dev_kernel<uint16_t><<<stream_grid(n), kThreads, 0, s>>>((uint16_t*)x, n, scale);
  else if (dtype == LZ_F16) scale_dev_kernel<_Float16><<<stream_grid(n), kThreads, 0, s>>>((_Float16*)x, n, scale);
  else if (dtype == LZ_F32) scale_dev_kernel<float><<<stream_grid(n), kThreads, 0, s>>>((float*)x, n, scale);
  else return lz_set_error(LZ_EINVAL, "lz_scale_dev: bad dtype %d", dtype);
  return lz_check_launch("lz_scale_dev");
}

LZ_EXPORT int lz_add_inplace(void* dst, const void* src, int dtype, int64_t n, void* stream) {
  LZ_REQUIRE(n >= 0, "lz_add_inplace: negative n");
  if (n == 0) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  if (dtype == LZ_BF16) add_inplace_kernel<uint16_t><<<stream_grid(n), kThreads, 0, s>>>((uint16_t*)dst, (const uint16_t*)src, n);
  else if (dtype == LZ_F16) add_inplace_kernel<_Float16><<<stream_grid(n), kThreads, 0, s>>>((_Float16*)dst, (const _Float16*)src, n);
  else if (dtype == LZ_F32) add_inplace_kernel<float><<<stream_grid(n), kThreads, 0, s>>>((float*)dst, (const float*)src, n);
  else return lz_set_error(LZ_EINVAL, "lz_add_inplace: bad dtype %d", dtype);
  return lz_check_launch("lz_add_inplace");
}

LZ_EXPORT int lz_scale_inplace(void* x, int dtype, int64_t n, float alpha, void* stream) {
  LZ_REQUIRE(n >= 0, "lz_scale_inplace: negative n");
  if (n == 0) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  if (dtype == LZ_BF16) scale_kernel<uint16_t><<<stream_grid(n), kThreads, 0, s>>>((uint16_t*)x, n, alpha);
  else if (dtype == LZ_F16) scale_kernel<_Float16><<<stream_grid(n), kThreads, 0, s>>>((_Float16*)x, n, alpha);
  else if (dtype == LZ_F32) scale_kernel<float><<<stream_grid(n), kThreads, 0, s>>>((float*)x, n, alpha);
  else return lz_set_error(LZ_EINVAL, "lz_scale_inplace: bad dtype %d", dtype);
  return lz_check_launch("lz_scale_inplace");
}

LZ_EXPORT int lz_mt_gather(const int64_t* table, int nseg, int src_dtype, void* dst, int dst_dtype, int64_t begin,
                           int64_t end, int accumulate, void* stream) {
  LZ_REQUIRE(table && nseg > 0 && begin <= end, "lz_mt_gather: bad arguments");
  LZ_REQUIRE(!accumulate || dst_dtype == LZ_F32, "lz_mt_gather: accumulate requires an fp32 destination");
  if (begin == end) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  const int grid = (int)std::min<int64_t>(lz_cdiv(end - begin, kChunk), (int64_t)lz_num_cus() * 8);
  if (src_dtype == LZ_BF16 && dst_dtype == LZ_BF16) mt_gather_kernel<uint16_t, uint16_t><<<grid, kThreads, 0, s>>>(table, nseg, (uint16_t*)dst, begin, end, 0);
  else if (src_dtype == LZ_BF16 && dst_dtype == LZ_F32) mt_gather_kernel<uint16_t, float><<<grid, kThreads, 0, s>>>(table, nseg, (float*)dst, begin, end, accumulate);
  else if (src_dtype == LZ_F32 && dst_dtype == LZ_F32) mt_gather_kernel<float, float><<<grid, kThreads, 0, s>>>(table, nseg, (float*)dst, begin, end, accumulate);
  else if (src_dtype == LZ_F32 && dst_dtype == LZ_BF16) mt_gather_kernel<float, uint16_t><<<grid, kThreads, 0, s>>>(table, nseg, (uint16_t*)dst, begin, end, 0);
  else return lz_set_error(LZ_EINVAL, "lz_mt_gather: bad dtypes");
  return lz_check_launch("lz_mt_gather");
}

LZ_EXPORT int lz_mt_scatter(const void* src, int src_dtype, const int64_t* table, int nseg, int dst_dtype, int64_t begin,
                            int64_t end, void* stream) {
  LZ_REQUIRE(table && nseg > 0 && begin <= end, "lz_mt_scatter: bad arguments");
  if (begin == end) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  const int grid = (int)std::min<int64_t>(lz_cdiv(end - begin, kChunk), (int64_t)lz_num_cus() * 8);
  if (src_dtype == LZ_F32 && dst_dtype == LZ_BF16) mt_scatter_kernel<float, uint16_t><<<grid, kThreads, 0, s>>>((const float*)src, table, nseg, begin, end);
  else if (src_dtype == LZ_F32 && dst_dtype == LZ_F32) mt_scatter_kernel<float, float><<<grid, kThreads, 0, s>>>((const float*)src, table, nseg, begin, end);
  else if (src_dtype == LZ_BF16 && dst_dtype == LZ_BF16) mt_scatter_kernel<uint16_t, uint16_t><<<grid, kThreads, 0, s>>>((const uint16_t*)src, table, nseg, begin, end);
  else if (src_dtype == LZ_BF16 && dst_dtype == LZ_F32) mt_scatter_kernel<uint16_t, float><<<grid, kThreads, 0, s>>>((const uint16_t*)src, table, nseg, begin, end);
  else return lz_set_error(LZ_EINVAL, "lz_mt_scatter: bad dtypes");
  return lz_check_launch("lz_mt_scatter");
}

// Same as lz_mt_gather / lz_mt_scatter with the {ptr, numel, flat_offset}
// records in host memory; they travel in the kernel arguments.
LZ_EXPORT int lz_mt_gather_host(const int64_t* host_table, int nseg, int src_dtype, void* dst, int dst_dtype,
                                int64_t begin, int64_t end, int accumulate, void* stream) {
  int rc = check_host_table(host_table, nseg);
  if (rc) return rc;
  LZ_REQUIRE(begin <= end && dst, "lz_mt_gather_host: bad range");
  LZ_REQUIRE(!accumulate || dst_dtype == LZ_F32, "lz_mt_gather_host: accumulate requires an fp32 destination");
  if (begin == end) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  if (src_dtype == LZ_BF16 && dst_dtype == LZ_BF16) return run_host_table<uint16_t, uint16_t>(0, host_table, nseg, dst, begin, end, 0, s);
  if (src_dtype == LZ_BF16 && dst_dtype == LZ_F32) return run_host_table<uint16_t, float>(0, host_table, nseg, dst, begin, end, accumulate, s);
  if (src_dtype == LZ_F32 && dst_dtype == LZ_F32) return run_host_table<float, float>(0, host_table, nseg, dst, begin, end, accumulate, s);
  if (src_dtype == LZ_F32 && dst_dtype == LZ_BF16) return run_host_table<float, uint16_t>(0, host_table, nseg, dst, begin, end, 0, s);
  if (src_dtype == LZ_F16 && dst_dtype == LZ_F32) return run_host_table<_Float16, float>(0, host_table, nseg, dst, begin, end, accumulate, s);
  return lz_set_error(LZ_EINVAL, "lz_mt_gather_host: bad dtypes");
}

LZ_EXPORT int lz_mt_scatter_host(const void* src, int src_dtype, const int64_t* host_table, int nseg, int dst_dtype,
                                 int64_t begin, int64_t end, void* stream) {
  int rc = check_host_table(host_table, nseg);
  if (rc) return rc;
  LZ_REQUIRE(begin <= end && src, "lz_mt_scatter_host: bad range");
  if (begin == end) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  void* srcp = const_cast<void*>(src);
  if (src_dtype == LZ_F32 && dst_dtype == LZ_BF16) return run_host_table<float, uint16_t>(1, host_table, nseg, srcp, begin, end, 0, s);
  if (src_dtype == LZ_F32 && dst_dtype == LZ_F32) return run_host_table<float, float>(1, host_table, nseg, srcp, begin, end, 0, s);
  if (src_dtype == LZ_BF16 && dst_dtype == LZ_BF16) return run_host_table<uint16_t, uint16_t>(1, host_table, nseg, srcp, begin, end, 0, s);
  if (src_dtype == LZ_BF16 && dst_dtype == LZ_F32) return run_host_table<uint16_t, float>(1, host_table, nseg, srcp, begin, end, 0, s);
  return lz_set_error(LZ_EINVAL, "lz_mt_scatter_host: bad dtypes");
}
