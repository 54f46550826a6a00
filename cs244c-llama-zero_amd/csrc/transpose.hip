// Batched 2-D transpose, dst[b1][b2][c][r] = src[b1][b2][r][c], through 64x64
// LDS tiles (padded rows so both the row-wise writes and the column-wise reads
// spread over the LDS banks).  Two batch levels let one launch transpose every
// (sequence, head) slice of a strided [B, S, heads, hd] projection.  Used to put
// an operand's reduction dimension innermost before an NT GEMM or an attention
// pass.  HBM-bound: 2 x element size per element.
#include "lz_common.h"

namespace {

constexpr int kTile = 64;

template <typename T>
__global__ void __launch_bounds__(256) transpose_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t nb2,
                                                         int64_t rows, int64_t cols, int64_t lds, int64_t sb1s,
                                                         int64_t sb2s, int64_t ldd, int64_t sb1d, int64_t sb2d) {
  __shared__ T tile[kTile][kTile + 2];
  const int64_t z = blockIdx.z;
  const int64_t b1 = z / nb2, b2 = z - b1 * nb2;
  const int64_t r0 = (int64_t)blockIdx.y * kTile, c0 = (int64_t)blockIdx.x * kTile;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const T* s = src + b1 * sb1s + b2 * sb2s;
  T* d = dst + b1 * sb1d + b2 * sb2d;
#pragma unroll
  for (int i = 0; i < kTile; i += 4) {
    const int64_t r = r0 + i + ty, c = c0 + tx;
    if (r < rows && c < cols) tile[i + ty][tx] = s[r * lds + c];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kTile; i += 4) {
    const int64_t c = c0 + i + ty, r = r0 + tx;
    if (r < rows && c < cols) d[c * ldd + r] = tile[tx][i + ty];
  }
}

template <typename T>
__global__ void __launch_bounds__(256) copy2d_kernel(const T* __restrict__ src, int64_t lds, T* __restrict__ dst,
                                                      int64_t ldd, int64_t rows, int64_t cols) {
  const int64_t total = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cols, c = i - r * cols;
    dst[r * ldd + c] = src[r * lds + c];
  }
}

// 16-byte chunks: thread x of row y copies chunk blockIdx.x*256 + x of that
// row (rows past gridDim.y are taken in steps of gridDim.y).  One chunk per
// thread and no loop over columns measured fastest for plain copies here
// (6.1-6.2 TB/s at 128 MB-2 GB); nontemporal loads keep the stream out of L2.
typedef unsigned int chunk16_t __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256) copy2d_vec_kernel(const chunk16_t* __restrict__ src, int64_t lds,
                                                          chunk16_t* __restrict__ dst, int64_t ldd, int64_t rows,
                                                          int64_t cols) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) dst[r * ldd + c] = __builtin_nontemporal_load(src + r * lds + c);
}

}  // namespace

// dst[r][c] = src[r][c] for a rows x cols window of two row-major matrices.
LZ_EXPORT int lz_copy2d(const void* src, int64_t lds, void* dst, int64_t ldd, int64_t rows, int64_t cols, int dtype,
                        void* stream) {
  LZ_REQUIRE(rows >= 0 && cols >= 0 && lds >= cols && ldd >= cols, "lz_copy2d: bad shape");
  if (rows == 0 || cols == 0) return LZ_OK;
  hipStream_t s = lz_stream(stream);
  LZ_REQUIRE(dtype == LZ_BF16 || dtype == LZ_F32 || dtype == LZ_F16, "lz_copy2d: bad dtype %d", dtype);
  const int64_t esz = lz_esize(dtype);  // a copy: the 16-bit formats move alike
  if (lz_aligned16(src) && lz_aligned16(dst) && (cols * esz) % 16 == 0 &&
      (lds * esz) % 16 == 0 && (ldd * esz) % 16 == 0) {
    int64_t vr = rows, vc = cols * esz / 16, vls = lds * esz / 16, vld = ldd * esz / 16;
    if (vls == vc && vld == vc) {  // both contiguous: one long row
      vc *= vr;
      vr = 1;
    }
    LZ_REQUIRE(lz_cdiv(vc, 256) < (1ll << 31), "lz_copy2d: too many columns");
    const dim3 grid((unsigned)lz_cdiv(vc, 256), (unsigned)std::min<int64_t>(vr, 65535));
    copy2d_vec_kernel<<<grid, 256, 0, s>>>((const chunk16_t*)src, vls, (chunk16_t*)dst, vld, vr, vc);
    return lz_check_launch("lz_copy2d");
  }
  const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(lz_cdiv(rows * cols, 256), (int64_t)lz_num_cus() * 16));
  if (dtype == LZ_F32) copy2d_kernel<float><<<grid, 256, 0, s>>>((const float*)src, lds, (float*)dst, ldd, rows, cols);
  else copy2d_kernel<uint16_t><<<grid, 256, 0, s>>>((const uint16_t*)src, lds, (uint16_t*)dst, ldd, rows, cols);
  return lz_check_launch("lz_copy2d");
}

LZ_EXPORT int lz_transpose(const void* src, void* dst, int dtype, int64_t nb1, int64_t nb2, int64_t rows, int64_t cols,
                           int64_t lds, int64_t sb1s, int64_t sb2s, int64_t ldd, int64_t sb1d, int64_t sb2d,
                           void* stream) {
  LZ_REQUIRE(nb1 >= 0 && nb2 >= 1 && rows >= 0 && cols >= 0 && lds >= cols && ldd >= rows, "lz_transpose: bad shape");
  if (nb1 == 0 || rows == 0 || cols == 0) return LZ_OK;
  LZ_REQUIRE(nb1 * nb2 < 65536, "lz_transpose: too many batches");
  LZ_REQUIRE(lz_cdiv(rows, kTile) < 65536, "lz_transpose: too many rows");
  dim3 grid((unsigned)lz_cdiv(cols, kTile), (unsigned)lz_cdiv(rows, kTile), (unsigned)(nb1 * nb2));
  hipStream_t s = lz_stream(stream);
  if (dtype == LZ_BF16 || dtype == LZ_F16)  // a permutation: the 16-bit formats move alike
    transpose_kernel<uint16_t><<<grid, 256, 0, s>>>((const uint16_t*)src, (uint16_t*)dst, nb2, rows, cols, lds, sb1s, sb2s,
                                                     ldd, sb1d, sb2d);
  else if (dtype == LZ_F32)
    transpose_kernel<float><<<grid, 256, 0, s>>>((const float*)src, (float*)dst, nb2, rows, cols, lds, sb1s, sb2s, ldd,
                                                  sb1d, sb2d);
  else
    return lz_set_error(LZ_EINVAL, "lz_transpose: bad dtype %d", dtype);
  return lz_check_launch("lz_transpose");
}
