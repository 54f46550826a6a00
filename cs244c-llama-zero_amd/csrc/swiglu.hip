// SwiGLU pointwise part (reference: model/llama.py:136-146):
//   h = silu(g) * u,   silu(g) = g / (1 + exp(-g))
// with the reference's rounding in the activation dtype: silu's result is
// rounded before the product, the product rounded again.  The backward
// follows autograd of the same two ops:
//   ds = r(dh * u),  du = r(dh * r(silu(g))),
//   dg = r(ds * sig * (1 + g * (1 - sig))).
// Gate and up may be two column ranges of one fused [T, 2*ffn] projection.
// HBM-bound: forward 6 B/element (read g,u; write h), backward 10 B/element.
// The bf16 vector kernels evaluate sigmoid with the hardware exp2/reciprocal
// (about 1 ulp in fp32, below the bf16 rounding of every output).
#include "lz_common.h"

namespace {

// 16-byte nontemporal load for operands that are streamed once (measured on
// [16384, 5632]: forward 17 % faster; together with the one-row-per-grid-row
// launch below, forward 106 -> 82 us and backward 180 -> 160 us).
__device__ __forceinline__ uint4 ntl16(const uint16_t* p) {
  typedef unsigned int v4u __attribute__((ext_vector_type(4)));
  const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

template <typename T>
__global__ void swiglu_fwd_kernel(const T* __restrict__ g, int64_t ldg, const T* __restrict__ u, int64_t ldu,
                                  T* __restrict__ h, int64_t ldh, int64_t rows, int64_t cols) {
  const int64_t total = rows * cols;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = idx / cols, c = idx - r * cols;
    const float gv = Elem<T>::load(g + r * ldg, c);
    const float uv = Elem<T>::load(u + r * ldu, c);
    const float s = Elem<T>::round(silu_f(gv));
    Elem<T>::store(h + r * ldh, c, s * uv);
  }
}


// Vector path: 8 bf16 per thread (16-byte accesses).  blockIdx.x covers a
// row's 16-byte chunks, blockIdx.y strides over rows, so no index division.
__global__ void __launch_bounds__(256) swiglu_fwd_bf16x8_kernel(const uint16_t* __restrict__ g, int64_t ldg,
                                                                const uint16_t* __restrict__ u, int64_t ldu,
                                                                uint16_t* __restrict__ h, int64_t ldh, int64_t rows,
                                                                int cpr) {
  const int cc = blockIdx.x * blockDim.x + threadIdx.x;
  if (cc >= cpr) return;
  const int64_t c = (int64_t)cc << 3;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    *reinterpret_cast<uint4*>(h + r * ldh + c) = swiglu_fwd8(ntl16(g + r * ldg + c), ntl16(u + r * ldu + c));
  }
}

template <typename T>
__device__ __forceinline__ void swiglu_bwd_elem(float gv, float uv, float dh, float& dg, float& du) {
  const float sig = 1.0f / (1.0f + expf(-gv));
  const float s = Elem<T>::round(gv / (1.0f + expf(-gv)));
  const float ds = Elem<T>::round(dh * uv);
  du = dh * s;
  dg = ds * sig * (1.0f + gv * (1.0f - sig));
}

template <typename T>
__global__ void swiglu_bwd_kernel(const T* __restrict__ g, int64_t ldg, const T* __restrict__ u, int64_t ldu,
                                  const T* __restrict__ dh, int64_t lddh, T* __restrict__ dg, int64_t lddg,
                                  T* __restrict__ du, int64_t lddu, int64_t rows, int64_t cols) {
  const int64_t total = rows * cols;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = idx / cols, c = idx - r * cols;
    float a, b;
    swiglu_bwd_elem<T>(Elem<T>::load(g + r * ldg, c), Elem<T>::load(u + r * ldu, c), Elem<T>::load(dh + r * lddh, c), a, b);
    Elem<T>::store(dg + r * lddg, c, a);
    Elem<T>::store(du + r * lddu, c, b);
  }
}

__global__ void __launch_bounds__(256) swiglu_bwd_bf16x8_kernel(
    const uint16_t* __restrict__ g, int64_t ldg, const uint16_t* __restrict__ u, int64_t ldu,
    const uint16_t* __restrict__ dh, int64_t lddh, uint16_t* __restrict__ dg, int64_t lddg, uint16_t* __restrict__ du,
    int64_t lddu, int64_t rows, int cpr) {
  const int cc = blockIdx.x * blockDim.x + threadIdx.x;
  if (cc >= cpr) return;
  const int64_t c = (int64_t)cc << 3;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const uint4 gv = ntl16(g + r * ldg + c);
    const uint4 uv = ntl16(u + r * ldu + c);
    const uint4 hv = ntl16(dh + r * lddh + c);
    uint4 gav, uav;
    swiglu_bwd8(gv, uv, hv, gav, uav);
    *reinterpret_cast<uint4*>(dg + r * lddg + c) = gav;
    *reinterpret_cast<uint4*>(du + r * lddu + c) = uav;
  }
}

// 2-D grid of the vector kernels: one row per grid row (rows past 65535 are
// taken in strides), so each thread handles one 8-element chunk per row and
// the hardware spreads the whole launch; measured faster than a grid sized to
// the CUs with each thread looping over rows.
inline dim3 vec_grid(int64_t rows, int cpr) {
  const int bx = (int)lz_cdiv(cpr, 256);
  return dim3((unsigned)bx, (unsigned)std::min<int64_t>(std::max<int64_t>(rows, 1), 65535));
}

inline int grid_for(int64_t n) {
  int64_t b = lz_cdiv(n, 256);
  int64_t cap = (int64_t)lz_num_cus() * 16;
  return (int)std::max<int64_t>(1, std::min(b, cap));
}

inline bool vec_ok(const void* p, int64_t ld) { return lz_aligned16(p) && (ld % 8) == 0; }

}  // namespace

LZ_EXPORT int lz_swiglu_fwd(const void* g, int64_t ldg, const void* u, int64_t ldu, void* h, int64_t ldh, int64_t rows,
                            int64_t cols, int dtype, void* stream) {
  LZ_REQUIRE(rows >= 0 && cols >= 0 && cols < ((int64_t)1 << 31) && ldg >= cols && ldu >= cols && ldh >= cols,
             "lz_swiglu_fwd: bad shape");
  if (rows == 0 || cols == 0) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  if (dtype == LZ_BF16) {
    if (cols % 8 == 0 && vec_ok(g, ldg) && vec_ok(u, ldu) && vec_ok(h, ldh))
      swiglu_fwd_bf16x8_kernel<<<vec_grid(rows, (int)(cols / 8)), 256, 0, s>>>((const uint16_t*)g, ldg, (const uint16_t*)u, ldu, (uint16_t*)h, ldh, rows, (int)(cols / 8));
    else
      swiglu_fwd_kernel<uint16_t><<<grid_for(rows * cols), 256, 0, s>>>((const uint16_t*)g, ldg, (const uint16_t*)u, ldu, (uint16_t*)h, ldh, rows, cols);
  } else if (dtype == LZ_F32) {
    swiglu_fwd_kernel<float><<<grid_for(rows * cols), 256, 0, s>>>((const float*)g, ldg, (const float*)u, ldu, (float*)h, ldh, rows, cols);
  } else if (dtype == LZ_F16) {
    swiglu_fwd_kernel<_Float16><<<grid_for(rows * cols), 256, 0, s>>>((const _Float16*)g, ldg, (const _Float16*)u, ldu, (_Float16*)h, ldh, rows, cols);
  } else {
    return lz_set_error(LZ_EINVAL, "lz_swiglu_fwd: bad dtype %d", dtype);
  }
  return lz_check_launch("lz_swiglu_fwd");
}

LZ_EXPORT int lz_swiglu_bwd(const void* g, int64_t ldg, const void* u, int64_t ldu, const void* dh, int64_t lddh,
                            void* dg, int64_t lddg, void* du, int64_t lddu, int64_t rows, int64_t cols, int dtype,
                            void* stream) {
  LZ_REQUIRE(rows >= 0 && cols >= 0 && cols < ((int64_t)1 << 31) && ldg >= cols && ldu >= cols && lddh >= cols &&
                 lddg >= cols && lddu >= cols,
             "lz_swiglu_bwd: bad shape");
  if (rows == 0 || cols == 0) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  if (dtype == LZ_BF16) {
    if (cols % 8 == 0 && vec_ok(g, ldg) && vec_ok(u, ldu) && vec_ok(dh, lddh) && vec_ok(dg, lddg) && vec_ok(du, lddu))
      swiglu_bwd_bf16x8_kernel<<<vec_grid(rows, (int)(cols / 8)), 256, 0, s>>>((const uint16_t*)g, ldg, (const uint16_t*)u, ldu, (const uint16_t*)dh, lddh, (uint16_t*)dg, lddg, (uint16_t*)du, lddu, rows, (int)(cols / 8));
    else
      swiglu_bwd_kernel<uint16_t><<<grid_for(rows * cols), 256, 0, s>>>((const uint16_t*)g, ldg, (const uint16_t*)u, ldu, (const uint16_t*)dh, lddh, (uint16_t*)dg, lddg, (uint16_t*)du, lddu, rows, cols);
  } else if (dtype == LZ_F32) {
    swiglu_bwd_kernel<float><<<grid_for(rows * cols), 256, 0, s>>>((const float*)g, ldg, (const float*)u, ldu, (const float*)dh, lddh, (float*)dg, lddg, (float*)du, lddu, rows, cols);
  } else if (dtype == LZ_F16) {
    swiglu_bwd_kernel<_Float16><<<grid_for(rows * cols), 256, 0, s>>>((const _Float16*)g, ldg, (const _Float16*)u, ldu, (const _Float16*)dh, lddh, (_Float16*)dg, lddg, (_Float16*)du, lddu, rows, cols);
  } else {
    return lz_set_error(LZ_EINVAL, "lz_swiglu_bwd: bad dtype %d", dtype);
  }
  return lz_check_launch("lz_swiglu_bwd");
}
