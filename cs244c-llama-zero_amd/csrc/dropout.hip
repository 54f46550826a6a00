// Dropout (reference: model/llama.py:146 and :213, nn.Dropout on the MLP's
// gated activations and on the token embeddings, in training mode):
//   y = x * keep / (1 - p),  keep ~ Bernoulli(1 - p) per element,
// the backward applying the same keep mask to the incoming gradient.  The
// mask is not stored: it is a function of (seed, element index) through the
// counter-based stream in lz_common.h, so the backward (and the ZeRO-3
// recompute, which replays the seed) regenerates it.  HBM-bound: 4 B/element
// in bf16.
#include <cmath>

#include "lz_common.h"

namespace {

template <typename T>
__global__ void __launch_bounds__(256) dropout_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t n,
                                                      uint32_t thresh, float scale, uint64_t seed) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float v = Elem<T>::load(x, i);
    Elem<T>::store(y, i, lz_keep(seed, (uint64_t)i, thresh) ? v * scale : 0.0f);
  }
}

// 8 bf16 per thread (16-byte accesses), elements 8c .. 8c+7.
__global__ void __launch_bounds__(256) dropout_bf16x8_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
                                                             int64_t nchunk, uint32_t thresh, float scale,
                                                             uint64_t seed) {
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < nchunk; c += (int64_t)gridDim.x * blockDim.x) {
    const uint4 v = *reinterpret_cast<const uint4*>(x + 8 * c);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint64_t i0 = (uint64_t)(8 * c + 2 * k);
      const float a = lz_keep(seed, i0, thresh) ? bf2f((uint16_t)(w[k] & 0xffff)) * scale : 0.0f;
      const float b = lz_keep(seed, i0 + 1, thresh) ? bf2f((uint16_t)(w[k] >> 16)) * scale : 0.0f;
      o[k] = pack_bf16x2(a, b);
    }
    *reinterpret_cast<uint4*>(y + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

__global__ void __launch_bounds__(256) dropout_mask_kernel(uint8_t* __restrict__ keep, int64_t n, uint32_t thresh,
                                                           uint64_t seed) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    keep[i] = lz_keep(seed, (uint64_t)i, thresh) ? 1 : 0;
}

unsigned grid_for(int64_t work) { return (unsigned)std::min<int64_t>(lz_cdiv(work, 256), 65536); }

uint32_t drop_thresh(float p) {
  const double t = std::ceil((double)p * 16777216.0);
  return (uint32_t)std::min(t, 16777216.0);
}

}  // namespace

// y = x * keep / (1 - p) over n contiguous elements (x == y allowed), keep
// from (seed, index); the backward is the same call on the gradient with the
// same seed.  p in [0, 1]; p == 1 zeroes y.
LZ_EXPORT int lz_dropout(const void* x, void* y, int64_t n, float p, uint64_t seed, int dtype, void* stream) {
  LZ_REQUIRE(n >= 0 && p >= 0.f && p <= 1.f, "lz_dropout: bad arguments (n %lld, p %g)", (long long)n, (double)p);
  if (n == 0) return LZ_OK;
  LZ_REQUIRE(x && y, "lz_dropout: null pointer");
  hipStream_t s = lz_stream(stream);
  const uint32_t thresh = drop_thresh(p);
  const float scale = p < 1.f ? 1.0f / (1.0f - p) : 0.f;
  if (dtype == LZ_BF16) {
    if (n % 8 == 0 && lz_aligned16(x) && lz_aligned16(y))
      dropout_bf16x8_kernel<<<grid_for(n / 8), 256, 0, s>>>((const uint16_t*)x, (uint16_t*)y, n / 8, thresh, scale, seed);
    else
      dropout_kernel<uint16_t><<<grid_for(n), 256, 0, s>>>((const uint16_t*)x, (uint16_t*)y, n, thresh, scale, seed);
  } else if (dtype == LZ_F16) {
    dropout_kernel<_Float16><<<grid_for(n), 256, 0, s>>>((const _Float16*)x, (_Float16*)y, n, thresh, scale, seed);
  } else if (dtype == LZ_F32) {
    dropout_kernel<float><<<grid_for(n), 256, 0, s>>>((const float*)x, (float*)y, n, thresh, scale, seed);
  } else {
    return lz_set_error(LZ_EINVAL, "lz_dropout: bad dtype %d", dtype);
  }
  return lz_check_launch("lz_dropout");
}

// The keep mask lz_dropout (and attention dropout) uses for these n
// elements: one byte each, 1 = kept.
LZ_EXPORT int lz_dropout_mask(uint8_t* keep, int64_t n, float p, uint64_t seed, void* stream) {
  LZ_REQUIRE(n >= 0 && p >= 0.f && p <= 1.f, "lz_dropout_mask: bad arguments");
  if (n == 0) return LZ_OK;
  LZ_REQUIRE(keep, "lz_dropout_mask: null pointer");
  dropout_mask_kernel<<<grid_for(n), 256, 0, lz_stream(stream)>>>(keep, n, drop_thresh(p), seed);
  return lz_check_launch("lz_dropout_mask");
}
