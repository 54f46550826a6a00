// bf16 "NT" GEMM on CDNA4 matrix cores:
//
//   C[M,N] = alpha * A[M,K] . B[N,K]^T  (+ beta * C)  (+ R)
//
// A and B are row-major with the reduction dimension K innermost, which is the
// layout of nn.Linear's forward (x . W^T, reference model/llama.py:81-84,
// 139-141, 178).  fp32 accumulation, bf16 or fp32 output, optional residual
// add (the block's `x + f(x)`, model/llama.py:158-159) and optional
// accumulation into an existing fp32 C (gradient accumulation).
//
// Tiling: a workgroup computes a BM x BN tile with 64-wide K steps staged
// through double-buffered LDS (rows padded by 16 bytes so the 16-byte fragment
// reads of 8 consecutive lanes hit distinct banks).  Each wave owns a
// (BM/WM) x (BN/WN) sub-tile made of 32x32 v_mfma_f32_32x32x16_bf16 tiles.
// The MFMA computes D = B_tile . A_tile^T so that each lane ends up holding 4
// consecutive output columns of one output row, which are stored as one 8- or
// 16-byte write.  Global loads for step k+1 are in flight while step k's MFMAs
// run.  Workgroup ids are remapped so that consecutive tiles of one M-band land
// on the same XCD (its L2 then serves the shared A rows).
#include "lz_common.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;                 // K elements per stage
constexpr int kRowBytes = kBK * 2 + 16; // padded LDS row (144 B)

struct GemmArgs {
  const uint16_t* A;
  const uint16_t* B;
  void* C;
  const uint16_t* R;
  int64_t lda, ldb, ldc, ldr;
  int64_t M, N, K;
  float alpha, beta;
  int c_f32;      // output dtype fp32 (else bf16)
  int vec_store;  // N, ldc, ldr multiples of 4 and pointers aligned
};

__device__ __forceinline__ void store_out4(const GemmArgs& g, int64_t m, int64_t n, const float (&v)[4]) {
  float o[4] = {v[0] * g.alpha, v[1] * g.alpha, v[2] * g.alpha, v[3] * g.alpha};
  if (g.vec_store && n + 3 < g.N) {
    if (g.c_f32) {
      float4* cp = reinterpret_cast<float4*>(static_cast<float*>(g.C) + m * g.ldc + n);
      if (g.beta != 0.f) {
        float4 c = *cp;
        o[0] = fmaf(g.beta, c.x, o[0]); o[1] = fmaf(g.beta, c.y, o[1]);
        o[2] = fmaf(g.beta, c.z, o[2]); o[3] = fmaf(g.beta, c.w, o[3]);
      }
      if (g.R) {
        uint2 r = *reinterpret_cast<const uint2*>(g.R + m * g.ldr + n);
        o[0] += bf2f(r.x & 0xffff); o[1] += bf2f(r.x >> 16); o[2] += bf2f(r.y & 0xffff); o[3] += bf2f(r.y >> 16);
      }
      *cp = make_float4(o[0], o[1], o[2], o[3]);
    } else {
      uint2* cp = reinterpret_cast<uint2*>(static_cast<uint16_t*>(g.C) + m * g.ldc + n);
      if (g.beta != 0.f) {
        uint2 c = *cp;
        o[0] = fmaf(g.beta, bf2f(c.x & 0xffff), o[0]); o[1] = fmaf(g.beta, bf2f(c.x >> 16), o[1]);
        o[2] = fmaf(g.beta, bf2f(c.y & 0xffff), o[2]); o[3] = fmaf(g.beta, bf2f(c.y >> 16), o[3]);
      }
      if (g.R) {
        uint2 r = *reinterpret_cast<const uint2*>(g.R + m * g.ldr + n);
        o[0] += bf2f(r.x & 0xffff); o[1] += bf2f(r.x >> 16); o[2] += bf2f(r.y & 0xffff); o[3] += bf2f(r.y >> 16);
      }
      uint2 w;
      w.x = (uint32_t)f2bf(o[0]) | ((uint32_t)f2bf(o[1]) << 16);
      w.y = (uint32_t)f2bf(o[2]) | ((uint32_t)f2bf(o[3]) << 16);
      *cp = w;
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t nn = n + e;
    if (nn >= g.N) break;
    float val = o[e];
    if (g.c_f32) {
      float* cp = static_cast<float*>(g.C) + m * g.ldc + nn;
      if (g.beta != 0.f) val = fmaf(g.beta, *cp, val);
      if (g.R) val += bf2f(g.R[m * g.ldr + nn]);
      *cp = val;
    } else {
      uint16_t* cp = static_cast<uint16_t*>(g.C) + m * g.ldc + nn;
      if (g.beta != 0.f) val = fmaf(g.beta, bf2f(*cp), val);
      if (g.R) val += bf2f(g.R[m * g.ldr + nn]);
      *cp = f2bf(val);
    }
  }
}

// Maps the linear workgroup id to a (tile_m, tile_n) pair.  Hardware places
// workgroup i on XCD i % 8; the remap gives each XCD a contiguous range of
// logical tiles, and the logical order walks groups of kGroupM M-tiles across
// all N-tiles so an XCD's concurrently running tiles share A rows and B rows.
__device__ __forceinline__ void tile_coords(int64_t tiles_m, int64_t tiles_n, int64_t& tm, int64_t& tn) {
  constexpr int kXcd = 8, kGroupM = 8;
  const int64_t nblk = tiles_m * tiles_n;
  int64_t pid = blockIdx.x;
  if (nblk % kXcd == 0) pid = (pid % kXcd) * (nblk / kXcd) + pid / kXcd;
  const int64_t per_group = (int64_t)kGroupM * tiles_n;
  const int64_t group = pid / per_group;
  const int64_t first_m = group * kGroupM;
  const int64_t gsize = min((int64_t)kGroupM, tiles_m - first_m);
  const int64_t in_group = pid - group * per_group;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

template <int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(64 * WM * WN) gemm_nt_kernel(GemmArgs g) {
  constexpr int kThreads = 64 * WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;      // wave sub-tile
  constexpr int FM = TM / 32, FN = TN / 32;      // 32x32 MFMA tiles per wave
  constexpr int kChunksA = BM * (kBK / 8) / kThreads;  // 16-byte chunks per thread per stage
  constexpr int kChunksB = BN * (kBK / 8) / kThreads;
  constexpr int kStageBytes = (BM + BN) * kRowBytes;
  static_assert(kChunksA * kThreads == BM * kBK / 8 && kChunksB * kThreads == BN * kBK / 8, "tile/thread mismatch");

  __shared__ __attribute__((aligned(16))) char smem[2 * kStageBytes];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t tiles_m = lz_cdiv(g.M, BM), tiles_n = lz_cdiv(g.N, BN);
  int64_t tm, tn;
  tile_coords(tiles_m, tiles_n, tm, tn);
  const int64_t m0 = tm * BM, n0 = tn * BN;
  const int64_t ktiles = lz_cdiv(g.K, kBK);

  // global->register staging
  uint4 ra[kChunksA], rb[kChunksB];
  auto gload = [&](int64_t kt) {
    const int64_t kbase = kt * kBK;
#pragma unroll
    for (int i = 0; i < kChunksA; ++i) {
      const int c = tid + i * kThreads;
      const int row = c >> 3, ch = c & 7;
      const int64_t gm = m0 + row, gk = kbase + ch * 8;
      ra[i] = (gm < g.M && gk < g.K) ? *reinterpret_cast<const uint4*>(g.A + gm * g.lda + gk) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kChunksB; ++i) {
      const int c = tid + i * kThreads;
      const int row = c >> 3, ch = c & 7;
      const int64_t gn = n0 + row, gk = kbase + ch * 8;
      rb[i] = (gn < g.N && gk < g.K) ? *reinterpret_cast<const uint4*>(g.B + gn * g.ldb + gk) : make_uint4(0, 0, 0, 0);
    }
  };
  auto sstore = [&](int stage) {
    char* As = smem + stage * kStageBytes;
    char* Bs = As + BM * kRowBytes;
#pragma unroll
    for (int i = 0; i < kChunksA; ++i) {
      const int c = tid + i * kThreads;
      *reinterpret_cast<uint4*>(As + (c >> 3) * kRowBytes + (c & 7) * 16) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < kChunksB; ++i) {
      const int c = tid + i * kThreads;
      *reinterpret_cast<uint4*>(Bs + (c >> 3) * kRowBytes + (c & 7) * 16) = rb[i];
    }
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  gload(0);
  sstore(0);
  __syncthreads();

  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * 16;  // byte offset of this lane's 8 K values

  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < ktiles) gload(kt + 1);
    const char* As = smem + cur * kStageBytes;
    const char* Bs = As + BM * kRowBytes;
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      bf16x8_t fa[FN], fb[FM];
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int row = wn * TN + j * 32 + frag_row;
        fa[j] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(Bs + row * kRowBytes + kk * 32 + frag_k));
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm * TM + i * 32 + frag_row;
        fb[i] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(As + row * kRowBytes + kk * 32 + frag_k));
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[j], fb[i], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < ktiles) sstore(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds output row m = (lane % 32) of each 32x32 tile and
  // columns n = 8*(r/4) + 4*(lane/32) + r%4.
  const int half = lane >> 5;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int64_t m = m0 + wm * TM + i * 32 + frag_row;
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t n = n0 + wn * TN + j * 32 + q * 8 + half * 4;
        if (n >= g.N) continue;
        const float v[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        store_out4(g, m, n, v);
      }
    }
  }
}

template <int BM, int BN, int WM, int WN>
int launch(const GemmArgs& g, hipStream_t s) {
  const int64_t tiles = lz_cdiv(g.M, BM) * lz_cdiv(g.N, BN);
  LZ_REQUIRE(tiles < (1ll << 31), "lz_gemm: too many tiles");
  gemm_nt_kernel<BM, BN, WM, WN><<<(unsigned)tiles, 64 * WM * WN, 0, s>>>(g);
  return lz_check_launch("lz_gemm_nt");
}

}  // namespace

// C = alpha * A . B^T (+ beta*C) (+ R).  A: [M,K] bf16 (lda), B: [N,K] bf16
// (ldb), C: [M,N] bf16 or fp32 (ldc), R: optional [M,N] bf16 (ldr).
// Requirements: K % 8 == 0, lda % 8 == 0, ldb % 8 == 0, A and B 16-byte aligned.
LZ_EXPORT int lz_gemm_nt(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, int c_dtype,
                         const void* R, int64_t ldr, int64_t M, int64_t N, int64_t K, float alpha, float beta,
                         void* stream) {
  LZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "lz_gemm_nt: negative shape");
  if (M == 0 || N == 0) return LZ_OK;
  LZ_REQUIRE(A && B && C, "lz_gemm_nt: null pointer");
  LZ_REQUIRE(K % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0, "lz_gemm_nt: K (%lld), lda, ldb must be multiples of 8",
             (long long)K);
  LZ_REQUIRE(lz_aligned16(A) && lz_aligned16(B), "lz_gemm_nt: A and B must be 16-byte aligned");
  LZ_REQUIRE(lda >= K && ldb >= K && ldc >= N && (R == nullptr || ldr >= N), "lz_gemm_nt: bad leading dimension");
  LZ_REQUIRE(c_dtype == LZ_BF16 || c_dtype == LZ_F32, "lz_gemm_nt: bad output dtype %d", c_dtype);
  GemmArgs g;
  g.A = (const uint16_t*)A;
  g.B = (const uint16_t*)B;
  g.C = C;
  g.R = (const uint16_t*)R;
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.ldr = ldr;
  g.M = M;
  g.N = N;
  g.K = K;
  g.alpha = alpha;
  g.beta = beta;
  g.c_f32 = c_dtype == LZ_F32;
  const int esz = g.c_f32 ? 4 : 2;
  g.vec_store = (N % 4 == 0) && (ldc % 4 == 0) && ((reinterpret_cast<uintptr_t>(C) & (4 * esz - 1)) == 0) &&
                (R == nullptr || ((ldr % 4 == 0) && (reinterpret_cast<uintptr_t>(R) & 7) == 0));
  hipStream_t s = lz_stream(stream);
  if (K == 0) {
    // nothing to reduce: C = beta*C + R handled by the epilogue with zero accumulators
  }
  const int64_t big_tiles = lz_cdiv(M, 256) * lz_cdiv(N, 256);
  if (big_tiles >= lz_num_cus()) return launch<256, 256, 2, 4>(g, s);
  return launch<128, 128, 2, 2>(g, s);
}
