// Shifted causal-LM cross entropy over a [rows, vocab] logits matrix
// (reference: model/llama.py:273-302, F.cross_entropy with ignore_index -100,
// computed in fp32 from the activation dtype as autocast does).
//
// Row r = b*seq + s is scored against labels[r + 1] when s < seq - 1 (the
// reference's logits[:, :-1] vs labels[:, 1:]); the last position of each
// sequence, ignore_index targets and out-of-range targets contribute nothing.
// With seq == 0 rows are scored against labels[r] (no shift).
//
// Forward: one workgroup per row, online log-sum-exp over 16-byte chunks
// (bf16 logits: in base 2 with the hardware exp2, about 1 ulp per term),
// writes lse[r] and the row loss (lse - x[target]); a single-block reduction
// then forms the mean deterministically.  Backward writes
// (softmax - onehot) * grad / count per element; it may run in place over the
// logits.  Both passes read the logits once: 2 B/element forward, 4 B/element
// backward in bf16.
#include "lz_common.h"

namespace {

constexpr int kThreads = 256;
constexpr float kLog2E = 1.4426950408889634f, kLn2 = 0.6931471805599453f;

__device__ __forceinline__ int64_t row_target(const int64_t* labels, int64_t r, int64_t seq, int64_t vocab,
                                              int64_t ignore_index) {
  int64_t t;
  if (seq > 0) {
    if ((r % seq) == seq - 1) return -1;
    t = labels[r + 1];
  } else {
    t = labels[r];
  }
  if (t == ignore_index || t < 0 || t >= vocab) return -1;
  return t;
}

template <typename T, bool kVec>
__global__ void __launch_bounds__(kThreads) ce_fwd_kernel(const T* __restrict__ logits, int64_t ld, int64_t rows, int64_t vocab,
                                                          const int64_t* __restrict__ labels, int64_t seq,
                                                          int64_t ignore_index, float* __restrict__ lse_out,
                                                          float* __restrict__ row_loss) {
  __shared__ float red[kThreads / 64];
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const T* x = logits + r * ld;
    float m = -INFINITY, s = 0.f;
    if (kVec) {
      // base-2 domain: u = x log2(e), s = sum 2^(u - m) with the hardware
      // exp2 (libm expf made this pass ALU-bound); converted back below
      const int64_t nchunk = vocab >> 3;
      // four 16-byte chunks per thread at a time, their loads issued
      // together, so enough bytes are in flight to stream the row at the
      // copy rate; the running max moves once per group of 32 values
      const uint4* xv = reinterpret_cast<const uint4*>(x);
      int64_t c = threadIdx.x;
      for (; c + 3 * kThreads < nchunk; c += 4 * kThreads) {
        uint4 raw[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) raw[u] = xv[c + u * kThreads];
        float v[32];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            v[8 * u + 2 * k] = bf2f(w[k] & 0xffff) * kLog2E;
            v[8 * u + 2 * k + 1] = bf2f(w[k] >> 16) * kLog2E;
          }
        }
        float cm = v[0];
#pragma unroll
        for (int k = 1; k < 32; ++k) cm = fmaxf(cm, v[k]);
        if (cm > m) {
          s = s * __builtin_amdgcn_exp2f(m - cm);
          m = cm;
        }
#pragma unroll
        for (int k = 0; k < 32; ++k) s += __builtin_amdgcn_exp2f(v[k] - m);
      }
      for (; c < nchunk; c += kThreads) {
        float v[8];
        const uint4 raw = xv[c];
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          v[2 * k] = bf2f(w[k] & 0xffff) * kLog2E;
          v[2 * k + 1] = bf2f(w[k] >> 16) * kLog2E;
        }
        float cm = v[0];
#pragma unroll
        for (int k = 1; k < 8; ++k) cm = fmaxf(cm, v[k]);
        if (cm > m) {
          s = s * __builtin_amdgcn_exp2f(m - cm);
          m = cm;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) s += __builtin_amdgcn_exp2f(v[k] - m);
      }
    } else {
      for (int64_t c = threadIdx.x; c < vocab; c += kThreads) {
        const float v = Elem<T>::load(x, c);
        if (v > m) {
          s = s * expf(m - v);
          m = v;
        }
        s += expf(v - m);
      }
    }
    const float M = block_max(m, red);
    const float part = (m == -INFINITY) ? 0.f : s * (kVec ? __builtin_amdgcn_exp2f(m - M) : expf(m - M));
    const float S = block_sum(part, red);
    if (threadIdx.x == 0) {
      const float lse = kVec ? (M + log2f(S)) * kLn2 : M + logf(S);
      lse_out[r] = lse;
      const int64_t t = row_target(labels, r, seq, vocab, ignore_index);
      row_loss[r] = t >= 0 ? lse - Elem<T>::load(x, t) : 0.f;
    }
    __syncthreads();
  }
}

// loss = sum(row_loss) / count  (count clamped to >= 1 when clamp != 0;
// otherwise 0/0 gives NaN, as F.cross_entropy's mean does with no targets).
__global__ void __launch_bounds__(1024) ce_reduce_kernel(const float* __restrict__ row_loss, const int64_t* __restrict__ labels,
                                                         int64_t rows, int64_t seq, int64_t vocab, int64_t ignore_index,
                                                         float* __restrict__ loss_out, float* __restrict__ count_out, int clamp) {
  __shared__ double red_s[16];
  __shared__ double red_c[16];
  double acc = 0.0, cnt = 0.0;
  for (int64_t r = threadIdx.x; r < rows; r += blockDim.x) {
    if (row_target(labels, r, seq, vocab, ignore_index) >= 0) {
      acc += (double)row_loss[r];
      cnt += 1.0;
    }
  }
  acc = wave_sum_d(acc);
  cnt = wave_sum_d(cnt);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) {
    red_s[wid] = acc;
    red_c[wid] = cnt;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double S = 0.0, C = 0.0;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) {
      S += red_s[i];
      C += red_c[i];
    }
    if (clamp && C < 1.0) C = 1.0;
    *loss_out = (float)(S / C);
    *count_out = (float)C;
  }
}

template <typename T, typename D, bool kVec>
__global__ void __launch_bounds__(kThreads) ce_bwd_kernel(const T* logits, int64_t ld, int64_t rows, int64_t vocab,
                                                          const int64_t* __restrict__ labels, int64_t seq,
                                                          int64_t ignore_index, const float* __restrict__ lse,
                                                          const float* __restrict__ grad_loss, const float* __restrict__ count,
                                                          D* dlogits, int64_t ldd) {
  const float scale = grad_loss[0] / count[0];
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const int64_t t = row_target(labels, r, seq, vocab, ignore_index);
    const T* x = logits + r * ld;
    D* d = dlogits + r * ldd;
    const float l = lse[r];
    if (kVec) {
      const int64_t nchunk = vocab >> 3;
      // 8 logits -> 8 gradients (d may alias x: every chunk is read before
      // it is written, by the same thread)
      auto grad8 = [&](const uint4& raw, int64_t c) {
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int64_t v0 = 8 * c + 2 * k;
          float g0 = 0.f, g1 = 0.f;
          if (t >= 0) {
            g0 = (__builtin_amdgcn_exp2f((bf2f(w[k] & 0xffff) - l) * kLog2E) - (v0 == t ? 1.f : 0.f)) * scale;
            g1 = (__builtin_amdgcn_exp2f((bf2f(w[k] >> 16) - l) * kLog2E) - (v0 + 1 == t ? 1.f : 0.f)) * scale;
          }
          o[k] = (uint32_t)f2bf(g0) | ((uint32_t)f2bf(g1) << 16);
        }
        return make_uint4(o[0], o[1], o[2], o[3]);
      };
      // four chunks per thread at a time, their loads issued together
      int64_t c = threadIdx.x;
      for (; c + 3 * kThreads < nchunk; c += 4 * kThreads) {
        uint4 raw[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) raw[u] = reinterpret_cast<const uint4*>(x)[c + u * kThreads];
#pragma unroll
        for (int u = 0; u < 4; ++u) reinterpret_cast<uint4*>(d)[c + u * kThreads] = grad8(raw[u], c + u * kThreads);
      }
      for (; c < nchunk; c += kThreads) reinterpret_cast<uint4*>(d)[c] = grad8(reinterpret_cast<const uint4*>(x)[c], c);
    } else {
      for (int64_t c = threadIdx.x; c < vocab; c += kThreads) {
        float g = 0.f;
        if (t >= 0) g = (expf(Elem<T>::load(x, c) - l) - (c == t ? 1.f : 0.f)) * scale;
        Elem<D>::store(d, c, g);
      }
    }
  }
}

inline int grid_rows(int64_t rows) { return (int)std::max<int64_t>(1, std::min<int64_t>(rows, (int64_t)lz_num_cus() * 32)); }

}  // namespace

LZ_EXPORT int lz_ce_fwd(const void* logits, int64_t ld, int64_t rows, int64_t vocab, int dtype, const int64_t* labels,
                        int64_t seq, int64_t ignore_index, float* lse, float* row_loss, void* stream) {
  LZ_REQUIRE(rows >= 0 && vocab > 0 && ld >= vocab && labels && lse && row_loss, "lz_ce_fwd: bad arguments");
  if (rows == 0) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  if (dtype == LZ_BF16) {
    if (vocab % 8 == 0 && ld % 8 == 0 && lz_aligned16(logits))
      ce_fwd_kernel<uint16_t, true><<<grid_rows(rows), kThreads, 0, s>>>((const uint16_t*)logits, ld, rows, vocab, labels, seq, ignore_index, lse, row_loss);
    else
      ce_fwd_kernel<uint16_t, false><<<grid_rows(rows), kThreads, 0, s>>>((const uint16_t*)logits, ld, rows, vocab, labels, seq, ignore_index, lse, row_loss);
  } else if (dtype == LZ_F32) {
    ce_fwd_kernel<float, false><<<grid_rows(rows), kThreads, 0, s>>>((const float*)logits, ld, rows, vocab, labels, seq, ignore_index, lse, row_loss);
  } else if (dtype == LZ_F16) {
    ce_fwd_kernel<_Float16, false><<<grid_rows(rows), kThreads, 0, s>>>((const _Float16*)logits, ld, rows, vocab, labels, seq, ignore_index, lse, row_loss);
  } else {
    return lz_set_error(LZ_EINVAL, "lz_ce_fwd: bad dtype %d", dtype);
  }
  return lz_check_launch("lz_ce_fwd");
}

LZ_EXPORT int lz_ce_reduce(const float* row_loss, const int64_t* labels, int64_t rows, int64_t seq, int64_t vocab,
                           int64_t ignore_index, float* loss_out, float* count_out, int clamp_count, void* stream) {
  LZ_REQUIRE(rows >= 0 && labels && row_loss && loss_out && count_out, "lz_ce_reduce: bad arguments");
  ce_reduce_kernel<<<1, 1024, 0, lz_stream(stream)>>>(row_loss, labels, rows, seq, vocab, ignore_index, loss_out, count_out,
                                                      clamp_count);
  return lz_check_launch("lz_ce_reduce");
}

LZ_EXPORT int lz_ce_bwd(const void* logits, int64_t ld, int64_t rows, int64_t vocab, int dtype, const int64_t* labels,
                        int64_t seq, int64_t ignore_index, const float* lse, const float* grad_loss, const float* count,
                        void* dlogits, int64_t ldd, int ddtype, void* stream) {
  LZ_REQUIRE(rows >= 0 && vocab > 0 && ld >= vocab && ldd >= vocab && labels && lse && grad_loss && count,
             "lz_ce_bwd: bad arguments");
  if (rows == 0) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  const int g = grid_rows(rows);
  if (dtype == LZ_BF16 && ddtype == LZ_BF16) {
    if (vocab % 8 == 0 && ld % 8 == 0 && ldd % 8 == 0 && lz_aligned16(logits) && lz_aligned16(dlogits))
      ce_bwd_kernel<uint16_t, uint16_t, true><<<g, kThreads, 0, s>>>((const uint16_t*)logits, ld, rows, vocab, labels, seq, ignore_index, lse, grad_loss, count, (uint16_t*)dlogits, ldd);
    else
      ce_bwd_kernel<uint16_t, uint16_t, false><<<g, kThreads, 0, s>>>((const uint16_t*)logits, ld, rows, vocab, labels, seq, ignore_index, lse, grad_loss, count, (uint16_t*)dlogits, ldd);
  } else if (dtype == LZ_F32 && ddtype == LZ_F32) {
    ce_bwd_kernel<float, float, false><<<g, kThreads, 0, s>>>((const float*)logits, ld, rows, vocab, labels, seq, ignore_index, lse, grad_loss, count, (float*)dlogits, ldd);
  } else if (dtype == LZ_BF16 && ddtype == LZ_F32) {
    ce_bwd_kernel<uint16_t, float, false><<<g, kThreads, 0, s>>>((const uint16_t*)logits, ld, rows, vocab, labels, seq, ignore_index, lse, grad_loss, count, (float*)dlogits, ldd);
  } else if (dtype == LZ_F16 && ddtype == LZ_F16) {
    ce_bwd_kernel<_Float16, _Float16, false><<<g, kThreads, 0, s>>>((const _Float16*)logits, ld, rows, vocab, labels, seq, ignore_index, lse, grad_loss, count, (_Float16*)dlogits, ldd);
  } else if (dtype == LZ_F16 && ddtype == LZ_F32) {
    ce_bwd_kernel<_Float16, float, false><<<g, kThreads, 0, s>>>((const _Float16*)logits, ld, rows, vocab, labels, seq, ignore_index, lse, grad_loss, count, (float*)dlogits, ldd);
  } else {
    return lz_set_error(LZ_EINVAL, "lz_ce_bwd: bad dtypes %d->%d", dtype, ddtype);
  }
  return lz_check_launch("lz_ce_bwd");
}
