// Token embedding gather and its gradient (reference: model/llama.py:174,212,
// nn.Embedding).
//
// Forward copies rows E[ids[t]] into out[t] (16-byte accesses).  An id outside
// [0, vocab) writes a zero row and raises a device flag instead of faulting.
// Backward scatters dout rows into an fp32 [vocab, dim] workspace with fp32
// atomics, then writes (or adds into) the gradient in the table's dtype.
#include "lz_common.h"

namespace {

template <typename T>
__global__ void embed_fwd_kernel(const int64_t* __restrict__ ids, int64_t ntok, const T* __restrict__ table, int64_t vocab,
                                 int64_t dim, T* __restrict__ out, int64_t ldo, int* __restrict__ bad_flag) {
  // one block-row of threads per token, grid-stride over tokens
  for (int64_t t = blockIdx.x; t < ntok; t += gridDim.x) {
    const int64_t id = ids[t];
    const bool ok = id >= 0 && id < vocab;
    if (!ok && threadIdx.x == 0 && bad_flag) atomicOr(bad_flag, 1);
    T* o = out + t * ldo;
    const T* src = table + (ok ? id : 0) * dim;
    for (int64_t c = threadIdx.x; c < dim; c += blockDim.x) o[c] = ok ? src[c] : T(0);
  }
}

__global__ void embed_fwd_vec_kernel(const int64_t* __restrict__ ids, int64_t ntok, const uint4* __restrict__ table,
                                     int64_t vocab, int64_t dim16, uint4* __restrict__ out, int64_t ldo16,
                                     int* __restrict__ bad_flag) {
  for (int64_t t = blockIdx.x; t < ntok; t += gridDim.x) {
    const int64_t id = ids[t];
    const bool ok = id >= 0 && id < vocab;
    if (!ok && threadIdx.x == 0 && bad_flag) atomicOr(bad_flag, 1);
    uint4* o = out + t * ldo16;
    const uint4* src = table + (ok ? id : 0) * dim16;
    for (int64_t c = threadIdx.x; c < dim16; c += blockDim.x) o[c] = ok ? src[c] : make_uint4(0, 0, 0, 0);
  }
}

template <typename T>
__global__ void embed_bwd_scatter_kernel(const int64_t* __restrict__ ids, int64_t ntok, const T* __restrict__ dout,
                                         int64_t ldo, int64_t vocab, int64_t dim, float* __restrict__ acc) {
  for (int64_t t = blockIdx.x; t < ntok; t += gridDim.x) {
    const int64_t id = ids[t];
    if (id < 0 || id >= vocab) continue;
    const T* g = dout + t * ldo;
    float* a = acc + id * dim;
    for (int64_t c = threadIdx.x; c < dim; c += blockDim.x) atomicAdd(a + c, Elem<T>::load(g, c));
  }
}

template <typename T>
__global__ void embed_bwd_finish_kernel(const float* __restrict__ acc, T* __restrict__ grad, int64_t n, int accumulate) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float v = acc[i];
    if (accumulate) v += Elem<T>::load(grad, i);
    Elem<T>::store(grad, i, v);
  }
}

__global__ void zero_f32_kernel(float* __restrict__ x, int64_t n) {
  const int64_t n4 = n >> 2;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x)
    reinterpret_cast<float4*>(x)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (blockIdx.x == 0)
    for (int64_t i = (n4 << 2) + threadIdx.x; i < n; i += blockDim.x) x[i] = 0.f;
}

inline int grid_cap(int64_t n) { return (int)std::max<int64_t>(1, std::min<int64_t>(n, (int64_t)lz_num_cus() * 16)); }

}  // namespace

LZ_EXPORT int lz_embedding_fwd(const int64_t* ids, int64_t ntok, const void* table, int64_t vocab, int64_t dim, void* out,
                               int64_t ldo, int dtype, int* bad_flag, void* stream) {
  LZ_REQUIRE(ntok >= 0 && vocab > 0 && dim > 0 && ldo >= dim, "lz_embedding_fwd: bad shape");
  if (ntok == 0) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  LZ_REQUIRE(dtype == LZ_BF16 || dtype == LZ_F32 || dtype == LZ_F16, "lz_embedding_fwd: bad dtype %d", dtype);
  const int esz = lz_esize(dtype);
  if ((dim * esz) % 16 == 0 && (ldo * esz) % 16 == 0 && lz_aligned16(table) && lz_aligned16(out)) {
    embed_fwd_vec_kernel<<<grid_cap(ntok), 128, 0, s>>>(ids, ntok, (const uint4*)table, vocab, dim * esz / 16, (uint4*)out,
                                                       ldo * esz / 16, bad_flag);
  } else if (dtype != LZ_F32) {  // a row copy: the 16-bit formats move alike
    embed_fwd_kernel<uint16_t><<<grid_cap(ntok), 128, 0, s>>>(ids, ntok, (const uint16_t*)table, vocab, dim, (uint16_t*)out, ldo, bad_flag);
  } else {
    embed_fwd_kernel<float><<<grid_cap(ntok), 128, 0, s>>>(ids, ntok, (const float*)table, vocab, dim, (float*)out, ldo, bad_flag);
  }
  return lz_check_launch("lz_embedding_fwd");
}

// workspace: vocab*dim fp32 (16-byte aligned).
LZ_EXPORT int lz_embedding_bwd(const int64_t* ids, int64_t ntok, const void* dout, int64_t ldo, int64_t vocab, int64_t dim,
                               void* grad, int accumulate, float* workspace, int dtype, void* stream) {
  LZ_REQUIRE(ntok >= 0 && vocab > 0 && dim > 0 && ldo >= dim, "lz_embedding_bwd: bad shape");
  LZ_REQUIRE(workspace && lz_aligned16(workspace), "lz_embedding_bwd: workspace must be 16-byte aligned");
  LZ_REQUIRE(dtype == LZ_BF16 || dtype == LZ_F32 || dtype == LZ_F16, "lz_embedding_bwd: bad dtype %d", dtype);
  hipStream_t s = lz_stream(stream);
  const int64_t n = vocab * dim;
  zero_f32_kernel<<<grid_cap(lz_cdiv(n / 4 + 1, 256)), 256, 0, s>>>(workspace, n);
  if (ntok > 0) {
    if (dtype == LZ_BF16) embed_bwd_scatter_kernel<uint16_t><<<grid_cap(ntok), 256, 0, s>>>(ids, ntok, (const uint16_t*)dout, ldo, vocab, dim, workspace);
    else if (dtype == LZ_F16) embed_bwd_scatter_kernel<_Float16><<<grid_cap(ntok), 256, 0, s>>>(ids, ntok, (const _Float16*)dout, ldo, vocab, dim, workspace);
    else embed_bwd_scatter_kernel<float><<<grid_cap(ntok), 256, 0, s>>>(ids, ntok, (const float*)dout, ldo, vocab, dim, workspace);
  }
  if (dtype == LZ_BF16) embed_bwd_finish_kernel<uint16_t><<<grid_cap(lz_cdiv(n, 256)), 256, 0, s>>>(workspace, (uint16_t*)grad, n, accumulate);
  else if (dtype == LZ_F16) embed_bwd_finish_kernel<_Float16><<<grid_cap(lz_cdiv(n, 256)), 256, 0, s>>>(workspace, (_Float16*)grad, n, accumulate);
  else embed_bwd_finish_kernel<float><<<grid_cap(lz_cdiv(n, 256)), 256, 0, s>>>(workspace, (float*)grad, n, accumulate);
  return lz_check_launch("lz_embedding_bwd");
}
