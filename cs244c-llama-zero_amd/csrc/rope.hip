// Rotary position embedding, NeoX half-split convention
// (reference: model/llama.py:25-39 rotate_half/apply_rotary_pos_emb and
// model/llama.py:42-69 RotaryEmbedding).
//
//   out = x * cos + rotate_half(x) * sin,  rotate_half(x) = cat(-x2, x1)
//
// The cos/sin table is built in fp32 (inv_freq = 1/theta^(2i/hd), angle =
// pos * inv_freq) and rounded to the activation dtype, as the reference's cache
// is.  The rotation reproduces the reference's per-operation rounding in the
// activation dtype: round(round(x*c) + round(r*s)).  Applied in place to heads
// stored as rows of `ld` elements, `nheads` heads of `hd` starting at column 0,
// so the q and k parts of a fused [T, (H+2KV)*hd] projection are rotated in one
// launch.  HBM-bound: 4 B/element read+write in bf16.
#include "lz_common.h"

namespace {

// The angle is formed in the dtype A of the module's inv_freq buffer, as the
// reference does after Module.to(dtype) has cast that buffer: the position
// (torch.arange in A), the product pos*inv_freq and cos/sin are each rounded
// to A; the table is then rounded to the activation dtype T.
template <typename T, typename A>
__global__ void rope_table_kernel(T* __restrict__ cos_t, T* __restrict__ sin_t, int64_t seq, int hd,
                                  const A* __restrict__ inv_freq) {
  const int half = hd / 2;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < seq * half; idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t pos = idx / half;
    const int i = (int)(idx % half);
    const float p = Elem<A>::round((float)pos);
    const float ang = Elem<A>::round(__fmul_rn(p, Elem<A>::load(inv_freq, i)));
    const float c = Elem<A>::round(cosf(ang)), s = Elem<A>::round(sinf(ang));
    Elem<T>::store(cos_t, pos * hd + i, c);
    Elem<T>::store(cos_t, pos * hd + i + half, c);
    Elem<T>::store(sin_t, pos * hd + i, s);
    Elem<T>::store(sin_t, pos * hd + i + half, s);
  }
}

__device__ __forceinline__ float mul_r(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_r(float a, float b) { return __fadd_rn(a, b); }

// One thread per (row, head, pair i in [0, hd/2)).
// Forward:  y1 = r(r(x1*c) + r(-x2*s)),   y2 = r(r(x2*c) + r(x1*s))
// Backward: g1 = r(r(d1*c) + r(d2*s)),    g2 = r(r(d2*c) + r(-(d1*s)))
template <typename T, bool kBwd>
__global__ void rope_kernel(T* __restrict__ x, int64_t ld, int64_t rows, int64_t seq, int nheads, int hd,
                            const T* __restrict__ cos_t, const T* __restrict__ sin_t, int64_t pos_offset) {
  // each product and the sum are rounded separately, as in the reference's
  // separate mul/add ops (this file is built with -ffp-contract=off)
  const int half = hd / 2;
  const int64_t per_row = (int64_t)nheads * half;
  const int64_t total = rows * per_row;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = idx / per_row;
    const int64_t rem = idx - row * per_row;
    const int head = (int)(rem / half);
    const int i = (int)(rem - (int64_t)head * half);
    const int64_t pos = row % seq + pos_offset;
    T* p = x + row * ld + (int64_t)head * hd;
    const float a = Elem<T>::load(p, i), b = Elem<T>::load(p, i + half);
    const float c1 = Elem<T>::load(cos_t, pos * hd + i), c2 = Elem<T>::load(cos_t, pos * hd + i + half);
    const float s1 = Elem<T>::load(sin_t, pos * hd + i), s2 = Elem<T>::load(sin_t, pos * hd + i + half);
    float o1, o2;
    if (!kBwd) {
      o1 = Elem<T>::round(add_r(Elem<T>::round(mul_r(a, c1)), Elem<T>::round(mul_r(-b, s1))));
      o2 = Elem<T>::round(add_r(Elem<T>::round(mul_r(b, c2)), Elem<T>::round(mul_r(a, s2))));
    } else {
      o1 = Elem<T>::round(add_r(Elem<T>::round(mul_r(a, c1)), Elem<T>::round(mul_r(b, s2))));
      o2 = Elem<T>::round(add_r(Elem<T>::round(mul_r(b, c2)), -Elem<T>::round(mul_r(a, s1))));
    }
    Elem<T>::store(p, i, o1);
    Elem<T>::store(p, i + half, o2);
  }
}

// Vectorized rotation: one thread per (row, group of V consecutive i < hd/2,
// four heads), V = 16 bytes of elements: the cos/sin vectors of the row's
// position are read once for the four heads, whose loads are in flight
// together.  Same per-element arithmetic as rope_kernel.
template <typename T, bool kBwd>
__device__ __forceinline__ void rope_vec_rotate(const uint4& av, const uint4& bv, const uint4& c1v, const uint4& c2v,
                                                const uint4& s1v, const uint4& s2v, uint4& o1v, uint4& o2v) {
  constexpr int V = 16 / sizeof(T);
  const T* a = reinterpret_cast<const T*>(&av);
  const T* b = reinterpret_cast<const T*>(&bv);
  const T* c1 = reinterpret_cast<const T*>(&c1v);
  const T* c2 = reinterpret_cast<const T*>(&c2v);
  const T* s1 = reinterpret_cast<const T*>(&s1v);
  const T* s2 = reinterpret_cast<const T*>(&s2v);
  T* o1 = reinterpret_cast<T*>(&o1v);
  T* o2 = reinterpret_cast<T*>(&o2v);
#pragma unroll
  for (int e = 0; e < V; ++e) {
    const float ae = Elem<T>::load(a, e), be = Elem<T>::load(b, e);
    float r1, r2;
    if (!kBwd) {
      r1 = Elem<T>::round(add_r(Elem<T>::round(mul_r(ae, Elem<T>::load(c1, e))), Elem<T>::round(mul_r(-be, Elem<T>::load(s1, e)))));
      r2 = Elem<T>::round(add_r(Elem<T>::round(mul_r(be, Elem<T>::load(c2, e))), Elem<T>::round(mul_r(ae, Elem<T>::load(s2, e)))));
    } else {
      r1 = Elem<T>::round(add_r(Elem<T>::round(mul_r(ae, Elem<T>::load(c1, e))), Elem<T>::round(mul_r(be, Elem<T>::load(s2, e)))));
      r2 = Elem<T>::round(add_r(Elem<T>::round(mul_r(be, Elem<T>::load(c2, e))), -Elem<T>::round(mul_r(ae, Elem<T>::load(s1, e)))));
    }
    Elem<T>::store(o1, e, r1);
    Elem<T>::store(o2, e, r2);
  }
}

template <typename T, bool kBwd>
__global__ void __launch_bounds__(256) rope_vec_kernel(T* __restrict__ x, int64_t ld, int rows, int seq, int nheads,
                                                       int hd, const T* __restrict__ cos_t, const T* __restrict__ sin_t,
                                                       int64_t pos_offset) {
  constexpr int V = 16 / sizeof(T);
  constexpr int kHeads = 4;  // heads per thread, in flight together
  const int half = hd / 2, groups = half / V;
  const int hquads = (nheads + kHeads - 1) / kHeads;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * groups * hquads) return;
  const int row = idx / (groups * hquads);
  const int rem = idx - row * (groups * hquads);
  const int hq = rem / groups;
  const int i = (rem - hq * groups) * V;
  const int64_t pos = row % seq + pos_offset;
  T* p = x + (int64_t)row * ld;
  const T* cp = cos_t + pos * hd;
  const T* sp = sin_t + pos * hd;
  const uint4 c1v = *reinterpret_cast<const uint4*>(cp + i), c2v = *reinterpret_cast<const uint4*>(cp + i + half);
  const uint4 s1v = *reinterpret_cast<const uint4*>(sp + i), s2v = *reinterpret_cast<const uint4*>(sp + i + half);
  int h = hq * kHeads;
  const int hend = min(nheads, h + kHeads);
  for (; h + kHeads <= hend; h += kHeads) {
    uint4 av[kHeads], bv[kHeads];
#pragma unroll
    for (int j = 0; j < kHeads; ++j) {
      av[j] = *reinterpret_cast<const uint4*>(p + (h + j) * hd + i);
      bv[j] = *reinterpret_cast<const uint4*>(p + (h + j) * hd + i + half);
    }
#pragma unroll
    for (int j = 0; j < kHeads; ++j) {
      uint4 o1v, o2v;
      rope_vec_rotate<T, kBwd>(av[j], bv[j], c1v, c2v, s1v, s2v, o1v, o2v);
      *reinterpret_cast<uint4*>(p + (h + j) * hd + i) = o1v;
      *reinterpret_cast<uint4*>(p + (h + j) * hd + i + half) = o2v;
    }
  }
  for (; h < hend; ++h) {
    const uint4 av = *reinterpret_cast<const uint4*>(p + h * hd + i);
    const uint4 bv = *reinterpret_cast<const uint4*>(p + h * hd + i + half);
    uint4 o1v, o2v;
    rope_vec_rotate<T, kBwd>(av, bv, c1v, c2v, s1v, s2v, o1v, o2v);
    *reinterpret_cast<uint4*>(p + h * hd + i) = o1v;
    *reinterpret_cast<uint4*>(p + h * hd + i + half) = o2v;
  }
}

inline int grid_for(int64_t n) {
  int64_t b = lz_cdiv(n, 256);
  int64_t cap = (int64_t)lz_num_cus() * 16;
  return (int)std::max<int64_t>(1, std::min(b, cap));
}

}  // namespace

// inv_freq: hd/2 device values of dtype freq_dtype (the module's buffer).
LZ_EXPORT int lz_rope_table(void* cos_t, void* sin_t, int dtype, int64_t seq, int64_t hd, const void* inv_freq,
                            int freq_dtype, void* stream) {
  LZ_REQUIRE(seq >= 0 && hd > 0 && hd % 2 == 0 && inv_freq, "lz_rope_table: bad arguments");
  if (seq == 0) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  const int g = grid_for(seq * hd / 2);
  LZ_REQUIRE(dtype >= LZ_F32 && dtype <= LZ_F16 && freq_dtype >= LZ_F32 && freq_dtype <= LZ_F16,
             "lz_rope_table: bad dtypes %d/%d", dtype, freq_dtype);
  const int key = dtype * 3 + freq_dtype;
  switch (key) {
    case LZ_F16 * 3 + LZ_F16:
      rope_table_kernel<_Float16, _Float16><<<g, 256, 0, s>>>((_Float16*)cos_t, (_Float16*)sin_t, seq, (int)hd, (const _Float16*)inv_freq);
      break;
    case LZ_F16 * 3 + LZ_F32:
      rope_table_kernel<_Float16, float><<<g, 256, 0, s>>>((_Float16*)cos_t, (_Float16*)sin_t, seq, (int)hd, (const float*)inv_freq);
      break;
    case LZ_BF16 * 3 + LZ_BF16:
      rope_table_kernel<uint16_t, uint16_t><<<g, 256, 0, s>>>((uint16_t*)cos_t, (uint16_t*)sin_t, seq, (int)hd, (const uint16_t*)inv_freq);
      break;
    case LZ_BF16 * 3 + LZ_F32:
      rope_table_kernel<uint16_t, float><<<g, 256, 0, s>>>((uint16_t*)cos_t, (uint16_t*)sin_t, seq, (int)hd, (const float*)inv_freq);
      break;
    case LZ_F32 * 3 + LZ_F32:
      rope_table_kernel<float, float><<<g, 256, 0, s>>>((float*)cos_t, (float*)sin_t, seq, (int)hd, (const float*)inv_freq);
      break;
    case LZ_F32 * 3 + LZ_BF16:
      rope_table_kernel<float, uint16_t><<<g, 256, 0, s>>>((float*)cos_t, (float*)sin_t, seq, (int)hd, (const uint16_t*)inv_freq);
      break;
    default:
      return lz_set_error(LZ_EINVAL, "lz_rope_table: bad dtypes %d/%d", dtype, freq_dtype);
  }
  return lz_check_launch("lz_rope_table");
}

// x: rows of `ld` elements; positions are row % seq + pos_offset; tables hold
// at least (seq + pos_offset) positions of hd entries.
LZ_EXPORT int lz_rope(void* x, int dtype, int64_t ld, int64_t rows, int64_t seq, int64_t nheads, int64_t hd,
                      const void* cos_t, const void* sin_t, int64_t pos_offset, int backward, void* stream) {
  LZ_REQUIRE(rows >= 0 && seq > 0 && nheads > 0 && hd > 0 && hd % 2 == 0, "lz_rope: bad shape");
  LZ_REQUIRE(ld >= nheads * hd, "lz_rope: leading dimension %lld < %lld", (long long)ld, (long long)(nheads * hd));
  if (rows == 0) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  LZ_REQUIRE(dtype == LZ_BF16 || dtype == LZ_F32 || dtype == LZ_F16, "lz_rope: bad dtype %d", dtype);
  const int esz = lz_esize(dtype), vec = 16 / esz;
  // (fp16 takes the element-wise kernel: the vector kernel's fp16 instance
  // does not compile with this file's flags)
  if (dtype != LZ_F16 && (hd / 2) % vec == 0 && (ld * esz) % 16 == 0 && lz_aligned16(x) &&
      lz_aligned16(cos_t) && lz_aligned16(sin_t)) {
    const int64_t work = rows * (hd / 2 / vec) * ((nheads + 3) / 4);
    LZ_REQUIRE(work < (1ll << 31) && seq < (1ll << 31), "lz_rope: too many rows");
    const unsigned grid = (unsigned)lz_cdiv(work, 256);
    const int r32 = (int)rows, s32 = (int)seq;
    if (dtype == LZ_BF16) {
      if (backward) rope_vec_kernel<uint16_t, true><<<grid, 256, 0, s>>>((uint16_t*)x, ld, r32, s32, (int)nheads, (int)hd, (const uint16_t*)cos_t, (const uint16_t*)sin_t, pos_offset);
      else rope_vec_kernel<uint16_t, false><<<grid, 256, 0, s>>>((uint16_t*)x, ld, r32, s32, (int)nheads, (int)hd, (const uint16_t*)cos_t, (const uint16_t*)sin_t, pos_offset);
    } else {
      if (backward) rope_vec_kernel<float, true><<<grid, 256, 0, s>>>((float*)x, ld, r32, s32, (int)nheads, (int)hd, (const float*)cos_t, (const float*)sin_t, pos_offset);
      else rope_vec_kernel<float, false><<<grid, 256, 0, s>>>((float*)x, ld, r32, s32, (int)nheads, (int)hd, (const float*)cos_t, (const float*)sin_t, pos_offset);
    }
    return lz_check_launch("lz_rope");
  }
  const int g = grid_for(rows * nheads * hd / 2);
  if (dtype == LZ_BF16) {
    if (backward) rope_kernel<uint16_t, true><<<g, 256, 0, s>>>((uint16_t*)x, ld, rows, seq, (int)nheads, (int)hd, (const uint16_t*)cos_t, (const uint16_t*)sin_t, pos_offset);
    else rope_kernel<uint16_t, false><<<g, 256, 0, s>>>((uint16_t*)x, ld, rows, seq, (int)nheads, (int)hd, (const uint16_t*)cos_t, (const uint16_t*)sin_t, pos_offset);
  } else if (dtype == LZ_F32) {
    if (backward) rope_kernel<float, true><<<g, 256, 0, s>>>((float*)x, ld, rows, seq, (int)nheads, (int)hd, (const float*)cos_t, (const float*)sin_t, pos_offset);
    else rope_kernel<float, false><<<g, 256, 0, s>>>((float*)x, ld, rows, seq, (int)nheads, (int)hd, (const float*)cos_t, (const float*)sin_t, pos_offset);
  } else if (dtype == LZ_F16) {
    if (backward) rope_kernel<_Float16, true><<<g, 256, 0, s>>>((_Float16*)x, ld, rows, seq, (int)nheads, (int)hd, (const _Float16*)cos_t, (const _Float16*)sin_t, pos_offset);
    else rope_kernel<_Float16, false><<<g, 256, 0, s>>>((_Float16*)x, ld, rows, seq, (int)nheads, (int)hd, (const _Float16*)cos_t, (const _Float16*)sin_t, pos_offset);
  } else {
    return lz_set_error(LZ_EINVAL, "lz_rope: bad dtype %d", dtype);
  }
  return lz_check_launch("lz_rope");
}
