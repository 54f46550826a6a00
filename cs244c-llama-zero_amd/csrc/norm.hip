// RMSNorm forward and backward (reference: model/llama.py:14-22).
//
//   y = x * rsqrt(mean(x^2) + eps) * w        (statistics in fp32)
//
// One 64-lane wavefront per row; each lane keeps its slice of the row in
// registers (8 elements per 16-byte access), so x is read once and y written
// once: 4 B/element in bf16.  The backward reads x and dy, writes dx (and an
// optional residual-gradient add), 6 B/element, and reduces dw through fp32
// partial rows (one per workgroup for bf16, per wave otherwise) and a
// two-level column sum.
#include <mutex>

#include "lz_common.h"

namespace {

constexpr int kRowsPerBlock = 4;  // one wave per row
constexpr int kThreads = 64 * kRowsPerBlock;


template <typename T>
struct Pack8;

// 16-byte nontemporal load: the rows are read once.  Against plain loads,
// on inputs that come from HBM as they do in a training step (a rotation of
// buffers larger than the 256 MB Infinity Cache): backward with the residual
// gradient 60.5 -> 57.1 us, forward 25.9 -> 24.7 us at [16384, 2048].
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
  typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));
  const v4u_t t = __builtin_nontemporal_load(reinterpret_cast<const v4u_t*>(p));
  return make_uint4(t[0], t[1], t[2], t[3]);
}

// 16-bit formats: T is the storage type (uint16_t = bf16, _Float16 = fp16),
// F the format policy.
template <typename T, typename F>
struct Pack8H {
  static __device__ __forceinline__ void unpack(const uint4& v, float (&r)[8]) {
    r[0] = F::to_f(v.x & 0xffff); r[1] = F::to_f(v.x >> 16);
    r[2] = F::to_f(v.y & 0xffff); r[3] = F::to_f(v.y >> 16);
    r[4] = F::to_f(v.z & 0xffff); r[5] = F::to_f(v.z >> 16);
    r[6] = F::to_f(v.w & 0xffff); r[7] = F::to_f(v.w >> 16);
  }
  static __device__ __forceinline__ void load(const T* p, float (&r)[8]) {
    unpack(*reinterpret_cast<const uint4*>(p), r);
  }
  static __device__ __forceinline__ void load_nt(const T* p, float (&r)[8]) { unpack(ld_nt16(p), r); }
  static __device__ __forceinline__ void store(T* p, const float (&r)[8]) {
    *reinterpret_cast<uint4*>(p) = make_uint4(F::pack2(r[0], r[1]), F::pack2(r[2], r[3]),
                                              F::pack2(r[4], r[5]), F::pack2(r[6], r[7]));
  }
};

template <>
struct Pack8<uint16_t> : Pack8H<uint16_t, FmtBF16> {};
template <>
struct Pack8<_Float16> : Pack8H<_Float16, FmtF16> {};

template <>
struct Pack8<float> {
  static __device__ __forceinline__ void load(const float* p, float (&r)[8]) {
    float4 a = reinterpret_cast<const float4*>(p)[0];
    float4 b = reinterpret_cast<const float4*>(p)[1];
    r[0] = a.x; r[1] = a.y; r[2] = a.z; r[3] = a.w;
    r[4] = b.x; r[5] = b.y; r[6] = b.z; r[7] = b.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&r)[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(r[0], r[1], r[2], r[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(r[4], r[5], r[6], r[7]);
  }
  static __device__ __forceinline__ void load_nt(const float* p, float (&r)[8]) { load(p, r); }
};

// NC = number of 8-element chunks per lane; cols == NC * 512 at most, and the
// row is processed as chunks c = lane + 64*j.
template <typename T, int NC>
__global__ void __launch_bounds__(kThreads) rmsnorm_fwd_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                                T* __restrict__ y, float* __restrict__ rstd_out,
                                                                int64_t rows, int cols, int64_t ldx, int64_t ldy,
                                                                float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nchunk = cols >> 3;
  const T* xr = x + row * ldx;
  float v[NC][8];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = lane + 64 * j;
    if (c < nchunk) {
      Pack8<T>::load_nt(xr + 8 * c, v[j]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[j][e], v[j][e], ss);
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)cols + eps);
  if (lane == 0 && rstd_out) rstd_out[row] = r;
  T* yr = y + row * ldy;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = lane + 64 * j;
    if (c < nchunk) {
      float wv[8], o[8];
      Pack8<T>::load(w + 8 * c, wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (v[j][e] * r) * wv[e];
      // plain stores: the next kernel (the QKV or gate|up GEMM) reads y at
      // once, and it then finds y in the caches (1B step 108.8 -> 108.4 ms
      // against nontemporal stores, which time faster only in isolation)
      Pack8<T>::store(yr + 8 * c, o);
    }
  }
}

// 16-bit backward (T = uint16_t for bf16, _Float16 for fp16): workgroup b owns rows [b*rpb, (b+1)*rpb), its wave w takes
// rows w, w+4, ... of that range and loads the next one (x, dy and the
// residual gradient) while it computes the current one.  The 4 waves' dw contributions are summed in LDS (in a fixed
// order) into one fp32 partial row per workgroup: dw_part[b][cols].
template <typename T, int NC>
__global__ void __launch_bounds__(kThreads) rmsnorm_bwd16_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const float* __restrict__ rstd,
    const T* __restrict__ dy, const T* __restrict__ dres, T* __restrict__ dx,
    float* __restrict__ dw_part, int64_t rows, int64_t rpb, int cols, int64_t ldx, int64_t lddy, int64_t lddx) {
  __shared__ float red[2][NC * 512];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nchunk = cols >> 3;
  const int64_t r0 = (int64_t)blockIdx.x * rpb, r1 = min(rows, r0 + rpb);
  float wv[NC][8], dwacc[NC][8];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = lane + 64 * j;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      dwacc[j][e] = 0.f;
      wv[j][e] = 0.f;
    }
    if (c < nchunk) Pack8<T>::load(w + 8 * c, wv[j]);
  }
  const float inv_n = 1.0f / (float)cols;
  uint4 xn[NC], gn[NC], rn[NC] = {};
  auto fetch = [&](int64_t row) {
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = lane + 64 * j;
      if (c < nchunk) {
        xn[j] = ld_nt16(x + row * ldx + 8 * c);
        gn[j] = ld_nt16(dy + row * lddy + 8 * c);
        if (dres) rn[j] = ld_nt16(dres + row * lddx + 8 * c);
      }
    }
  };
  int64_t row = r0 + wave;
  if (row < r1) fetch(row);
  for (; row < r1; row += kRowsPerBlock) {
    uint4 xc[NC], gc[NC], rc[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      xc[j] = xn[j];
      gc[j] = gn[j];
      rc[j] = rn[j];
    }
    if (row + kRowsPerBlock < r1) fetch(row + kRowsPerBlock);
    const float r = rstd[row];
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      if (lane + 64 * j < nchunk) {
        float xv[8], gv[8];
        Pack8<T>::unpack(xc[j], xv);
        Pack8<T>::unpack(gc[j], gv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          dot = fmaf(gv[e] * wv[j][e], xv[e], dot);
          dwacc[j][e] = fmaf(gv[e], xv[e] * r, dwacc[j][e]);
        }
      }
    }
    dot = wave_sum(dot);
    const float coef = dot * r * r * r * inv_n;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = lane + 64 * j;
      if (c < nchunk) {
        float xv[8], gv[8], o[8];
        Pack8<T>::unpack(xc[j], xv);
        Pack8<T>::unpack(gc[j], gv);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = r * wv[j][e] * gv[e] - coef * xv[e];
        if (dres) {
          float rv[8];
          Pack8<T>::unpack(rc[j], rv);
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] += rv[e];
        }
        Pack8<T>::store(dx + row * lddx + 8 * c, o);
      }
    }
  }
  // dw: waves 2,3 park their sums, waves 0,1 add them; wave 1 parks, wave 0
  // adds and writes the workgroup's partial row.
  auto park = [&](int slot) {
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = lane + 64 * j;
      if (c < nchunk)
#pragma unroll
        for (int e = 0; e < 8; ++e) red[slot][8 * c + e] = dwacc[j][e];
    }
  };
  auto take = [&](int slot) {
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = lane + 64 * j;
      if (c < nchunk)
#pragma unroll
        for (int e = 0; e < 8; ++e) dwacc[j][e] += red[slot][8 * c + e];
    }
  };
  if (wave >= 2) park(wave - 2);
  __syncthreads();
  if (wave < 2) take(wave);
  __syncthreads();
  if (wave == 1) park(0);
  __syncthreads();
  if (wave == 0) {
    take(0);
    float* part = dw_part + (int64_t)blockIdx.x * cols;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = lane + 64 * j;
      if (c < nchunk) {
        reinterpret_cast<float4*>(part + 8 * c)[0] = make_float4(dwacc[j][0], dwacc[j][1], dwacc[j][2], dwacc[j][3]);
        reinterpret_cast<float4*>(part + 8 * c)[1] = make_float4(dwacc[j][4], dwacc[j][5], dwacc[j][6], dwacc[j][7]);
      }
    }
  }
}

// Generic path for any cols (scalar accesses, two passes over the row).
template <typename T>
__global__ void __launch_bounds__(kThreads) rmsnorm_fwd_scalar_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                                       T* __restrict__ y, float* __restrict__ rstd_out,
                                                                       int64_t rows, int cols, int64_t ldx, int64_t ldy,
                                                                       float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * ldx;
  float ss = 0.f;
  for (int c = lane; c < cols; c += 64) {
    float t = Elem<T>::load(xr, c);
    ss = fmaf(t, t, ss);
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)cols + eps);
  if (lane == 0 && rstd_out) rstd_out[row] = r;
  T* yr = y + row * ldy;
  for (int c = lane; c < cols; c += 64) Elem<T>::store(yr, c, (Elem<T>::load(xr, c) * r) * Elem<T>::load(w, c));
}

// Backward.  Each wave walks rows row = wave_id, wave_id + nwaves, ... and keeps
// its dw contribution per owned column in registers; at the end it writes one
// fp32 partial row (dw_part[wave_id][cols]).
template <typename T, int NC>
__global__ void __launch_bounds__(kThreads) rmsnorm_bwd_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                                const float* __restrict__ rstd, const T* __restrict__ dy,
                                                                const T* __restrict__ dres, T* __restrict__ dx,
                                                                float* __restrict__ dw_part, int64_t rows, int cols,
                                                                int64_t ldx, int64_t lddy, int64_t lddx) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * kRowsPerBlock;
  const int nchunk = cols >> 3;
  float wv[NC][8];
  float dwacc[NC][8];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = lane + 64 * j;
#pragma unroll
    for (int e = 0; e < 8; ++e) dwacc[j][e] = 0.f;
    if (c < nchunk) Pack8<T>::load(w + 8 * c, wv[j]);
  }
  const float inv_n = 1.0f / (float)cols;
  for (int64_t row = wave; row < rows; row += nwaves) {
    const float r = rstd[row];
    float xv[NC][8], gv[NC][8];
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = lane + 64 * j;
      if (c < nchunk) {
        Pack8<T>::load(x + row * ldx + 8 * c, xv[j]);
        Pack8<T>::load(dy + row * lddy + 8 * c, gv[j]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          dot = fmaf(gv[j][e] * wv[j][e], xv[j][e], dot);
          dwacc[j][e] = fmaf(gv[j][e], xv[j][e] * r, dwacc[j][e]);
        }
      }
    }
    dot = wave_sum(dot);
    const float coef = dot * r * r * r * inv_n;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = lane + 64 * j;
      if (c < nchunk) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = r * wv[j][e] * gv[j][e] - coef * xv[j][e];
        if (dres) {
          float rv[8];
          Pack8<T>::load(dres + row * lddx + 8 * c, rv);
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] += rv[e];
        }
        Pack8<T>::store(dx + row * lddx + 8 * c, o);
      }
    }
  }
  float* part = dw_part + wave * cols;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = lane + 64 * j;
    if (c < nchunk) {
      reinterpret_cast<float4*>(part + 8 * c)[0] = make_float4(dwacc[j][0], dwacc[j][1], dwacc[j][2], dwacc[j][3]);
      reinterpret_cast<float4*>(part + 8 * c)[1] = make_float4(dwacc[j][4], dwacc[j][5], dwacc[j][6], dwacc[j][7]);
    }
  }
}

template <typename T>
__global__ void __launch_bounds__(kThreads) rmsnorm_bwd_scalar_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                                       const float* __restrict__ rstd, const T* __restrict__ dy,
                                                                       const T* __restrict__ dres, T* __restrict__ dx,
                                                                       float* __restrict__ dw_part, int64_t rows, int cols,
                                                                       int64_t ldx, int64_t lddy, int64_t lddx) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * kRowsPerBlock;
  float* part = dw_part + wave * cols;
  for (int c = lane; c < cols; c += 64) part[c] = 0.f;
  const float inv_n = 1.0f / (float)cols;
  for (int64_t row = wave; row < rows; row += nwaves) {
    const float r = rstd[row];
    float dot = 0.f;
    for (int c = lane; c < cols; c += 64)
      dot = fmaf(Elem<T>::load(dy + row * lddy, c) * Elem<T>::load(w, c), Elem<T>::load(x + row * ldx, c), dot);
    dot = wave_sum(dot);
    const float coef = dot * r * r * r * inv_n;
    for (int c = lane; c < cols; c += 64) {
      const float xv = Elem<T>::load(x + row * ldx, c), gv = Elem<T>::load(dy + row * lddy, c);
      float o = r * Elem<T>::load(w, c) * gv - coef * xv;
      if (dres) o += Elem<T>::load(dres + row * lddx, c);
      Elem<T>::store(dx + row * lddx, c, o);
      part[c] += gv * (xv * r);
    }
  }
}

// dw reduction over the per-wave partial rows, in two parallel levels:
// (column block of 64) x (slice of the partial rows) workgroups sum their
// slice with 4 rows of 64 coalesced lanes, then one pass adds the slices.
constexpr int kSlices = 16;

__global__ void __launch_bounds__(256) dw_slice_kernel(const float* __restrict__ part, int64_t nparts, int cols,
                                                        float* __restrict__ slices) {
  __shared__ float red[4][64];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + tx;
  const int64_t per = lz_cdiv(nparts, kSlices);
  const int64_t p0 = (int64_t)blockIdx.y * per, p1 = min(p0 + per, nparts);
  float s = 0.f;
  if (c < cols)
    for (int64_t p = p0 + ty; p < p1; p += 4) s += part[p * cols + c];
  red[ty][tx] = s;
  __syncthreads();
  if (ty == 0 && c < cols) slices[(int64_t)blockIdx.y * cols + c] = red[0][tx] + red[1][tx] + red[2][tx] + red[3][tx];
}

template <typename T>
__global__ void dw_final_kernel(const float* __restrict__ slices, int cols, T* __restrict__ dw, int accumulate) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < kSlices; ++k) s += slices[(int64_t)k * cols + c];
  if (accumulate) s += Elem<T>::load(dw, c);
  Elem<T>::store(dw, c, s);
}

// dw from the partial rows in one launch (cols % 4 == 0): each workgroup owns
// 32 columns; its 256 threads are 8 column quads (16-byte reads) x 32 row
// groups, each summing every 32nd partial row in order, then the 32 row-group
// sums are added in a fixed order.  Deterministic: no atomics, and the order
// does not depend on scheduling.
constexpr int kColsumCols = 32, kColsumGroups = 32;

template <typename T>
__global__ void __launch_bounds__(256) dw_colsum_kernel(const float* __restrict__ part, int64_t nparts, int cols,
                                                        T* __restrict__ dw, int accumulate) {
  __shared__ float4 red[kColsumGroups][kColsumCols / 4];
  const int cq = threadIdx.x % (kColsumCols / 4), rg = threadIdx.x / (kColsumCols / 4);
  const int c = blockIdx.x * kColsumCols + 4 * cq;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  if (c < cols) {
    int64_t p = rg;
    // sixteen partial rows in flight per thread (one round trip for the 512
    // partial rows of a 2048-column backward), then four, then one; the
    // additions follow p in every case, so the sum's order is fixed
    for (; p + 15 * kColsumGroups < nparts; p += 16 * kColsumGroups) {
      float4 v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = *reinterpret_cast<const float4*>(part + (p + u * kColsumGroups) * cols + c);
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        s.x += v[u].x;
        s.y += v[u].y;
        s.z += v[u].z;
        s.w += v[u].w;
      }
    }
    for (; p + 3 * kColsumGroups < nparts; p += 4 * kColsumGroups) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const float4*>(part + (p + u * kColsumGroups) * cols + c);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        s.x += v[u].x;
        s.y += v[u].y;
        s.z += v[u].z;
        s.w += v[u].w;
      }
    }
    for (; p < nparts; p += kColsumGroups) {
      const float4 v = *reinterpret_cast<const float4*>(part + p * cols + c);
      s.x += v.x;
      s.y += v.y;
      s.z += v.z;
      s.w += v.w;
    }
  }
  red[rg][cq] = s;
  __syncthreads();
  if (rg == 0 && c < cols) {
    float4 t = red[0][cq];
    for (int k = 1; k < kColsumGroups; ++k) {
      const float4 v = red[k][cq];
      t.x += v.x;
      t.y += v.y;
      t.z += v.z;
      t.w += v.w;
    }
    const float o[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) Elem<T>::store(dw, c + e, accumulate ? o[e] + Elem<T>::load(dw, c + e) : o[e]);
  }
}

// Column sums of `nparts` fp32 partial rows into dw (+= when accumulate).
template <typename T>
int dw_from_partials(const float* part, int64_t nparts, int cols, T* dw, int accumulate, float* slices,
                     hipStream_t s) {
  if (cols % 4 == 0) {
    dw_colsum_kernel<T><<<(unsigned)lz_cdiv(cols, kColsumCols), 256, 0, s>>>(part, nparts, cols, dw, accumulate);
  } else {
    dw_slice_kernel<<<dim3((unsigned)lz_cdiv(cols, 64), kSlices), 256, 0, s>>>(part, nparts, cols, slices);
    dw_final_kernel<T><<<(int)lz_cdiv(cols, 256), 256, 0, s>>>(slices, cols, dw, accumulate);
  }
  return lz_check_launch("lz_rmsnorm_bwd(dw)");
}

// bf16 vector backward: number of workgroups (one dw partial row each), one
// resident round of them (the register footprint grows with cols: 8, 4, 2, 1
// workgroups per CU for cols <= 512, 1024, 2048, 4096).
inline int64_t bwd_blocks(int64_t rows, int64_t cols) {
  const int per_cu = cols <= 512 ? 8 : cols <= 1024 ? 4 : cols <= 2048 ? 2 : 1;
  return std::max<int64_t>(1, std::min<int64_t>((int64_t)lz_num_cus() * per_cu, lz_cdiv(rows, kRowsPerBlock)));
}

inline int64_t bwd_waves(int64_t rows) {
  // two workgroups (8 waves) per compute unit, at most one wave per row
  int64_t n = std::min<int64_t>((int64_t)lz_num_cus() * 2 * kRowsPerBlock, std::max<int64_t>(rows, kRowsPerBlock));
  return std::max<int64_t>(kRowsPerBlock, (n / kRowsPerBlock) * kRowsPerBlock);
}

// Workspace bytes of one backward on the path its shape and layout take.
template <typename T>
bool bwd_vec(const void* x, const void* w, const void* dy, const void* dres, const void* dx, int64_t cols, int64_t ldx,
             int64_t lddy, int64_t lddx) {
  return cols % 8 == 0 && lz_aligned16(x) && lz_aligned16(w) && lz_aligned16(dy) && lz_aligned16(dx) &&
         (dres == nullptr || lz_aligned16(dres)) && (ldx * (int64_t)sizeof(T)) % 16 == 0 &&
         (lddy * (int64_t)sizeof(T)) % 16 == 0 && (lddx * (int64_t)sizeof(T)) % 16 == 0;
}

template <typename T>
int64_t bwd_bytes(bool vec, int64_t rows, int64_t cols) {
  if (sizeof(T) == 2 && vec && cols <= 4096) return (bwd_blocks(rows, cols) + kSlices) * cols * 4;
  return (bwd_waves(rows) + kSlices) * cols * 4;
}

template <typename T>
int fwd_dispatch(const void* x, const void* w, void* y, float* rstd, int64_t rows, int cols, int64_t ldx, int64_t ldy,
                 float eps, hipStream_t s) {
  const int grid = (int)lz_cdiv(rows, kRowsPerBlock);
  const bool vec = cols % 8 == 0 && lz_aligned16(x) && lz_aligned16(w) && lz_aligned16(y) &&
                   (ldx * (int64_t)sizeof(T)) % 16 == 0 && (ldy * (int64_t)sizeof(T)) % 16 == 0;
  const T* xp = (const T*)x;
  const T* wp = (const T*)w;
  T* yp = (T*)y;
  if (vec && cols <= 512) rmsnorm_fwd_kernel<T, 1><<<grid, kThreads, 0, s>>>(xp, wp, yp, rstd, rows, cols, ldx, ldy, eps);
  else if (vec && cols <= 1024) rmsnorm_fwd_kernel<T, 2><<<grid, kThreads, 0, s>>>(xp, wp, yp, rstd, rows, cols, ldx, ldy, eps);
  else if (vec && cols <= 2048) rmsnorm_fwd_kernel<T, 4><<<grid, kThreads, 0, s>>>(xp, wp, yp, rstd, rows, cols, ldx, ldy, eps);
  else if (vec && cols <= 4096) rmsnorm_fwd_kernel<T, 8><<<grid, kThreads, 0, s>>>(xp, wp, yp, rstd, rows, cols, ldx, ldy, eps);
  else rmsnorm_fwd_scalar_kernel<T><<<grid, kThreads, 0, s>>>(xp, wp, yp, rstd, rows, cols, ldx, ldy, eps);
  return lz_check_launch("lz_rmsnorm_fwd");
}

template <typename T>
int bwd_dispatch(const void* x, const void* w, const float* rstd, const void* dy, const void* dres, void* dx, void* dw,
                 int dw_accumulate, float* ws, int64_t ws_bytes, int64_t rows, int cols, int64_t ldx, int64_t lddy,
                 int64_t lddx, hipStream_t s) {
  // workspace: one fp32 partial row per wave (per workgroup on the bf16
  // vector path), then kSlices rows of slice sums
  const bool vec = cols % 8 == 0 && lz_aligned16(x) && lz_aligned16(w) && lz_aligned16(dy) && lz_aligned16(dx) &&
                   (dres == nullptr || lz_aligned16(dres)) && (ldx * (int64_t)sizeof(T)) % 16 == 0 &&
                   (lddy * (int64_t)sizeof(T)) % 16 == 0 && (lddx * (int64_t)sizeof(T)) % 16 == 0;
  const T *xp = (const T*)x, *wp = (const T*)w, *gp = (const T*)dy, *rp = (const T*)dres;
  T* dxp = (T*)dx;
  if constexpr (sizeof(T) == 2) {
    if (vec && cols <= 4096) {
      const int64_t nblk = bwd_blocks(rows, cols), rpb = lz_cdiv(rows, nblk);
      LZ_REQUIRE(ws_bytes >= (nblk + kSlices) * (int64_t)cols * 4, "lz_rmsnorm_bwd: workspace too small (%lld bytes)",
                 (long long)ws_bytes);
      const unsigned grid = (unsigned)nblk;
      if (cols <= 512) rmsnorm_bwd16_kernel<T, 1><<<grid, kThreads, 0, s>>>(xp, wp, rstd, gp, rp, dxp, ws, rows, rpb, cols, ldx, lddy, lddx);
      else if (cols <= 1024) rmsnorm_bwd16_kernel<T, 2><<<grid, kThreads, 0, s>>>(xp, wp, rstd, gp, rp, dxp, ws, rows, rpb, cols, ldx, lddy, lddx);
      else if (cols <= 2048) rmsnorm_bwd16_kernel<T, 4><<<grid, kThreads, 0, s>>>(xp, wp, rstd, gp, rp, dxp, ws, rows, rpb, cols, ldx, lddy, lddx);
      else rmsnorm_bwd16_kernel<T, 8><<<grid, kThreads, 0, s>>>(xp, wp, rstd, gp, rp, dxp, ws, rows, rpb, cols, ldx, lddy, lddx);
      int rc = lz_check_launch("lz_rmsnorm_bwd");
      if (rc) return rc;
      if (dw) rc = dw_from_partials<T>(ws, nblk, cols, (T*)dw, dw_accumulate, ws + nblk * (int64_t)cols, s);
      return rc;
    }
  }
  const int64_t nwaves = bwd_waves(rows);
  LZ_REQUIRE(ws_bytes >= (nwaves + kSlices) * (int64_t)cols * 4, "lz_rmsnorm_bwd: workspace too small (%lld bytes)",
             (long long)ws_bytes);
  const int grid = (int)(nwaves / kRowsPerBlock);
  if (vec && cols <= 512) rmsnorm_bwd_kernel<T, 1><<<grid, kThreads, 0, s>>>(xp, wp, rstd, gp, rp, dxp, ws, rows, cols, ldx, lddy, lddx);
  else if (vec && cols <= 1024) rmsnorm_bwd_kernel<T, 2><<<grid, kThreads, 0, s>>>(xp, wp, rstd, gp, rp, dxp, ws, rows, cols, ldx, lddy, lddx);
  else if (vec && cols <= 2048) rmsnorm_bwd_kernel<T, 4><<<grid, kThreads, 0, s>>>(xp, wp, rstd, gp, rp, dxp, ws, rows, cols, ldx, lddy, lddx);
  else if (vec && cols <= 4096) rmsnorm_bwd_kernel<T, 8><<<grid, kThreads, 0, s>>>(xp, wp, rstd, gp, rp, dxp, ws, rows, cols, ldx, lddy, lddx);
  else rmsnorm_bwd_scalar_kernel<T><<<grid, kThreads, 0, s>>>(xp, wp, rstd, gp, rp, dxp, ws, rows, cols, ldx, lddy, lddx);
  int rc = lz_check_launch("lz_rmsnorm_bwd");
  if (rc) return rc;
  if (dw) rc = dw_from_partials<T>(ws, nwaves, cols, (T*)dw, dw_accumulate, ws + nwaves * (int64_t)cols, s);
  return rc;
}

}  // namespace

LZ_EXPORT int lz_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd, int dtype, int64_t rows, int64_t cols,
                             int64_t ldx, int64_t ldy, float eps, void* stream) {
  LZ_REQUIRE(rows >= 0 && cols > 0 && cols < (1 << 30), "lz_rmsnorm_fwd: bad shape");
  LZ_REQUIRE(ldx >= cols && ldy >= cols, "lz_rmsnorm_fwd: bad leading dimension");
  if (rows == 0) return LZ_OK;
  if (dtype == LZ_BF16) return fwd_dispatch<uint16_t>(x, w, y, rstd, rows, (int)cols, ldx, ldy, eps, lz_stream(stream));
  if (dtype == LZ_F32) return fwd_dispatch<float>(x, w, y, rstd, rows, (int)cols, ldx, ldy, eps, lz_stream(stream));
  if (dtype == LZ_F16) return fwd_dispatch<_Float16>(x, w, y, rstd, rows, (int)cols, ldx, ldy, eps, lz_stream(stream));
  return lz_set_error(LZ_EINVAL, "lz_rmsnorm_fwd: bad dtype %d", dtype);
}

// Workspace bytes the backward wants for its dw partials.
LZ_EXPORT int64_t lz_rmsnorm_bwd_workspace(int64_t rows, int64_t cols) {
  return (std::max(bwd_waves(rows), bwd_blocks(rows, cols)) + kSlices) * cols * 4;
}

LZ_EXPORT int lz_rmsnorm_bwd(const void* x, const void* w, const float* rstd, const void* dy, const void* dres, void* dx,
                             void* dw, int dw_accumulate, void* workspace, int64_t workspace_bytes, int dtype, int64_t rows,
                             int64_t cols, int64_t ldx, int64_t lddy, int64_t lddx, void* stream) {
  LZ_REQUIRE(rows >= 0 && cols > 0 && cols < (1 << 30), "lz_rmsnorm_bwd: bad shape");
  LZ_REQUIRE(ldx >= cols && lddy >= cols && lddx >= cols, "lz_rmsnorm_bwd: bad leading dimension");
  LZ_REQUIRE(workspace != nullptr, "lz_rmsnorm_bwd: null workspace");
  if (rows == 0) return LZ_OK;
  if (dtype == LZ_BF16)
    return bwd_dispatch<uint16_t>(x, w, rstd, dy, dres, dx, dw, dw_accumulate, (float*)workspace, workspace_bytes, rows,
                                  (int)cols, ldx, lddy, lddx, lz_stream(stream));
  if (dtype == LZ_F32)
    return bwd_dispatch<float>(x, w, rstd, dy, dres, dx, dw, dw_accumulate, (float*)workspace, workspace_bytes, rows,
                               (int)cols, ldx, lddy, lddx, lz_stream(stream));
  if (dtype == LZ_F16)
    return bwd_dispatch<_Float16>(x, w, rstd, dy, dres, dx, dw, dw_accumulate, (float*)workspace, workspace_bytes,
                                  rows, (int)cols, ldx, lddy, lddx, lz_stream(stream));
  return lz_set_error(LZ_EINVAL, "lz_rmsnorm_bwd: bad dtype %d", dtype);
}

// ---------------------------------------------------------------------------
// Backward without a caller workspace, for callers that cannot allocate
// device memory (code under HIP graph capture, serving loops, harnesses that
// forbid allocation).  The dw partial rows live in `scratch`, a fixed array of
// kScratchBytes per device that stays allocated until the process ends.
// Every call writes the partial rows it reads, so nothing in it has to start
// at zero.  Every call on a device shares that device's array, so calls that
// overlap in time on one device (other streams, other threads) race.
// ---------------------------------------------------------------------------
constexpr int64_t kScratchBytes = 8ll << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch` (the host-side symbol is a stand-in,
// not a device address), looked up once per device.
int scratch_for_device(float** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return lz_set_error(LZ_ERUNTIME, "lz_rmsnorm_bwd_noalloc: no current device (%d)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return lz_set_error(LZ_ERUNTIME, "lz_rmsnorm_bwd_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                          hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return LZ_OK;
}

}  // namespace

namespace {

template <typename T>
int bwd_noalloc(const void* x, const void* w, const float* rstd, const void* dy, const void* dres, void* dx, void* dw,
                int dw_accumulate, int64_t rows, int64_t cols, int64_t ldx, int64_t lddy, int64_t lddx, void* stream) {
  const int64_t need = bwd_bytes<T>(bwd_vec<T>(x, w, dy, dres, dx, cols, ldx, lddy, lddx), rows, cols);
  LZ_REQUIRE(need <= kScratchBytes,
             "lz_rmsnorm_bwd_noalloc: rows %lld x cols %lld need %lld bytes of scratch, more than its %lld",
             (long long)rows, (long long)cols, (long long)need, (long long)kScratchBytes);
  float* ws = nullptr;
  const int rc = scratch_for_device(&ws);
  if (rc) return rc;
  return bwd_dispatch<T>(x, w, rstd, dy, dres, dx, dw, dw_accumulate, ws, kScratchBytes, rows, (int)cols, ldx, lddy,
                         lddx, lz_stream(stream));
}

}  // namespace

// lz_rmsnorm_bwd with the library's own scratch instead of a workspace:
// same arguments without workspace/workspace_bytes, same dtypes (bf16, fp32,
// fp16), same results bit for bit.  Shapes whose workspace
// (lz_rmsnorm_bwd_workspace for the path taken) exceeds the scratch are
// refused; 16-bit rows of up to 4096 columns fit at any row count.
LZ_EXPORT int lz_rmsnorm_bwd_noalloc(const void* x, const void* w, const float* rstd, const void* dy, const void* dres,
                                     void* dx, void* dw, int dw_accumulate, int dtype, int64_t rows, int64_t cols,
                                     int64_t ldx, int64_t lddy, int64_t lddx, void* stream) {
  LZ_REQUIRE(rows >= 0 && cols > 0 && cols < (1 << 30), "lz_rmsnorm_bwd_noalloc: bad shape");
  LZ_REQUIRE(ldx >= cols && lddy >= cols && lddx >= cols, "lz_rmsnorm_bwd_noalloc: bad leading dimension");
  LZ_REQUIRE(dtype == LZ_BF16 || dtype == LZ_F32 || dtype == LZ_F16, "lz_rmsnorm_bwd_noalloc: bad dtype %d", dtype);
  if (rows == 0) return LZ_OK;
  if (dtype == LZ_BF16)
    return bwd_noalloc<uint16_t>(x, w, rstd, dy, dres, dx, dw, dw_accumulate, rows, cols, ldx, lddy, lddx, stream);
  if (dtype == LZ_F16)
    return bwd_noalloc<_Float16>(x, w, rstd, dy, dres, dx, dw, dw_accumulate, rows, cols, ldx, lddy, lddx, stream);
  return bwd_noalloc<float>(x, w, rstd, dy, dres, dx, dw, dw_accumulate, rows, cols, ldx, lddy, lddx, stream);
}
