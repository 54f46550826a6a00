// fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x2_f32):
//
//   C[M,N] = alpha * sum_k A(m,k) B(n,k)  (+ beta * C)  (+ R)
//
// The float32 twin of the bf16 product in gemm.hip, for models kept in fp32
// (the reference's `--dtype float32`, train.py:148-160 and
// train_zero.py:74,150-164, where nn.Linear runs in fp32).  Same operand
// layouts: an operand is K-major (A(m,k) = A[m*lda + k]) or M/N-major
// (A(m,k) = A[k*lda + m]), so forward, input-gradient and weight-gradient
// products read the stored tensors directly.  Products and sums stay fp32
// (gfx950 has no reduced-precision fp32 mode), so results are within a few
// fp32 ulps of the exact product; any M, N, K and leading dimension work:
// rows past M/N and K past the end are zero-filled in LDS, stores are masked.
//
// Tiling: a 256-thread workgroup (4 waves, 2 x 2) owns a 128 x 128 tile,
// each wave 64 x 64 as 2 x 2 blocks of 32 x 32 MFMA accumulators.  K moves
// in 32-deep stages through double-buffered LDS, K-major rows padded to 36
// floats (16-byte fragment reads stay aligned).  The two 32-lane halves of a
// wave feed the MFMA's two K slots; half h takes K = h*16 + s of the stage at
// MFMA step s, so every lane reads its A and B fragments of four steps with
// one 16-byte LDS read each.  The next stage's global loads are in flight
// while the current stage's MFMAs run.
//
// Split-K: a product with few output tiles (under 192 of the 256 CUs busy)
// and a long K (a language-model head's input gradient reduces over the
// vocabulary) is cut into K slices of whole stages, one grid layer each; the
// slices write fp32 partial tiles into a workspace and a second kernel sums
// them in slice order, then applies alpha, beta*C and R as the unsplit
// epilogue does.  The result does not depend on timing.
#include "lz_common.h"

namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kTile = 128;          // rows of A (M) and of B (N) per workgroup
constexpr int kBK = 32;             // K per stage
constexpr int kRow = kBK + 4;       // padded LDS row, floats
constexpr int kThreads = 256;
constexpr int kStage = 2 * kTile * kRow;  // floats per stage (A tile then B tile)

struct F32Args {
  const float* A;
  const float* B;
  void* C;
  const float* R;
  int64_t lda, ldb, ldc, ldr;
  int64_t M, N, K;
  float alpha, beta;
  int c_f32;   // fp32 output (else bf16)
  int a_vec;   // A rows 16-byte aligned (16-byte global loads)
  int b_vec;
  int64_t kper;  // K per grid layer (a multiple of kBK when split)
  int64_t slab;  // > 0: layer z writes raw fp32 partials at C + z * slab
};

struct Plan {
  int splits;
  int64_t kper;
};

Plan make_plan(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = lz_cdiv(M, kTile) * lz_cdiv(N, kTile);
  Plan p{1, K};
  if (tiles >= 192 || K < 4 * kBK) return p;
  int64_t splits = std::min<int64_t>({lz_cdiv(256, tiles), K / (2 * kBK), 64});
  if (splits < 2) return p;
  p.kper = lz_cdiv(lz_cdiv(K, splits), kBK) * kBK;
  p.splits = (int)lz_cdiv(K, p.kper);
  if (p.splits < 2) p = Plan{1, K};
  return p;
}

int64_t plan_workspace(const Plan& p, int64_t M, int64_t N) {
  return p.splits > 1 ? (int64_t)p.splits * M * N * (int64_t)sizeof(float) : 0;
}

// Global -> registers for one operand tile: kTile rows of M (or N) x kBK of K.
// Each thread holds 4 float4 of the tile.
template <bool KMAJOR>
struct TileLoad {
  float4 v[4];

  __device__ __forceinline__ void load(const float* X, int64_t ld, int64_t rows, int64_t K, int64_t r0, int64_t k0,
                                       bool vec) {
    const int t = threadIdx.x;
    if (KMAJOR) {
      // 8 threads per row, 4 consecutive K each: row p*32 + t/8, K (t%8)*4
      const int kc = (t & 7) * 4;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int64_t r = r0 + p * 32 + (t >> 3);
        const int64_t k = k0 + kc;
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < rows && k < K) {
          const float* src = X + r * ld + k;
          if (vec && k + 4 <= K) {
            x = *reinterpret_cast<const float4*>(src);
          } else {
            x.x = src[0];
            if (k + 1 < K) x.y = src[1];
            if (k + 2 < K) x.z = src[2];
            if (k + 3 < K) x.w = src[3];
          }
        }
        v[p] = x;
      }
    } else {
      // 32 threads per K row, 4 consecutive rows each: K row p*8 + t/32
      const int rc = (t & 31) * 4;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int64_t k = k0 + p * 8 + (t >> 5);
        const int64_t r = r0 + rc;
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k < K && r < rows) {
          const float* src = X + k * ld + r;
          if (vec && r + 4 <= rows) {
            x = *reinterpret_cast<const float4*>(src);
          } else {
            x.x = src[0];
            if (r + 1 < rows) x.y = src[1];
            if (r + 2 < rows) x.z = src[2];
            if (r + 3 < rows) x.w = src[3];
          }
        }
        v[p] = x;
      }
    }
  }

  // Registers -> K-major LDS rows (dst = this operand's kTile x kRow block).
  __device__ __forceinline__ void store(float* dst) const {
    const int t = threadIdx.x;
    if (KMAJOR) {
      const int kc = (t & 7) * 4;
#pragma unroll
      for (int p = 0; p < 4; ++p) *reinterpret_cast<float4*>(dst + (p * 32 + (t >> 3)) * kRow + kc) = v[p];
    } else {
      const int rc = (t & 31) * 4;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int kr = p * 8 + (t >> 5);
        dst[(rc + 0) * kRow + kr] = v[p].x;
        dst[(rc + 1) * kRow + kr] = v[p].y;
        dst[(rc + 2) * kRow + kr] = v[p].z;
        dst[(rc + 3) * kRow + kr] = v[p].w;
      }
    }
  }
};

template <bool AK, bool BK>
__global__ void __launch_bounds__(kThreads) gemm_f32_kernel(F32Args g) {
  __shared__ __attribute__((aligned(16))) float lds[2 * kStage];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 31, h = lane >> 5;
  const int64_t m0 = (int64_t)blockIdx.y * kTile, n0 = (int64_t)blockIdx.x * kTile;
  const int64_t kbeg = (int64_t)blockIdx.z * g.kper, kend = min(g.K, kbeg + g.kper);

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int64_t nk = kend > kbeg ? lz_cdiv(kend - kbeg, kBK) : 0;
  TileLoad<AK> la;
  TileLoad<BK> lb;
  if (nk > 0) {
    la.load(g.A, g.lda, g.M, kend, m0, kbeg, g.a_vec);
    lb.load(g.B, g.ldb, g.N, kend, n0, kbeg, g.b_vec);
    la.store(lds);
    lb.store(lds + kTile * kRow);
    __syncthreads();
  }
  for (int64_t kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) {
      la.load(g.A, g.lda, g.M, kend, m0, kbeg + (kt + 1) * kBK, g.a_vec);
      lb.load(g.B, g.ldb, g.N, kend, n0, kbeg + (kt + 1) * kBK, g.b_vec);
    }
    const float* As = lds + (kt & 1) * kStage;
    const float* Bs = As + kTile * kRow;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      float4 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const float4*>(As + (wm * 64 + i * 32 + li) * kRow + h * 16 + s4 * 4);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const float4*>(Bs + (wn * 64 + j * 32 + li) * kRow + h * 16 + s4 * 4);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].x, b[j].x, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].y, b[j].y, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].z, b[j].z, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].w, b[j].w, acc[i][j], 0, 0, 0);
        }
    }
    if (more) {
      // the other buffer was last read before the previous barrier
      float* nxt = lds + ((kt + 1) & 1) * kStage;
      la.store(nxt);
      lb.store(nxt + kTile * kRow);
    }
    __syncthreads();
  }

  // Accumulator register r of lane (li, h) in block (i, j) holds
  // C[m][n] with m = 8*(r/4) + 4*h + r%4 and n = li inside the 32 x 32 block:
  // each store instruction writes two 128-byte row segments.
  if (g.slab > 0) {
    float* part = static_cast<float*>(g.C) + (int64_t)blockIdx.z * g.slab;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t n = n0 + wn * 64 + j * 32 + li;
        if (n >= g.N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          if (m < g.M) part[m * g.N + n] = acc[i][j][r];
        }
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t n = n0 + wn * 64 + j * 32 + li;
      if (n >= g.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (m >= g.M) continue;
        float val = acc[i][j][r] * g.alpha;
        if (g.c_f32) {
          float* cp = static_cast<float*>(g.C) + m * g.ldc + n;
          if (g.beta != 0.f) val = fmaf(g.beta, *cp, val);
          if (g.R) val += g.R[m * g.ldr + n];
          *cp = val;
        } else {
          uint16_t* cp = static_cast<uint16_t*>(g.C) + m * g.ldc + n;
          if (g.beta != 0.f) val = fmaf(g.beta, bf2f(*cp), val);
          if (g.R) val += g.R[m * g.ldr + n];
          *cp = f2bf(val);
        }
      }
    }
}

// C = alpha * sum_z part[z] (+ beta*C) (+ R), the slices summed in order.
__global__ void __launch_bounds__(256) splitk_reduce_f32_kernel(F32Args g, const float* __restrict__ part,
                                                                 int splits) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= g.M * g.N) return;
  const int64_t m = i / g.N, n = i - m * g.N;
  float acc = 0.f;
  for (int z = 0; z < splits; ++z) acc += part[z * g.slab + i];
  float val = acc * g.alpha;
  if (g.c_f32) {
    float* cp = static_cast<float*>(g.C) + m * g.ldc + n;
    if (g.beta != 0.f) val = fmaf(g.beta, *cp, val);
    if (g.R) val += g.R[m * g.ldr + n];
    *cp = val;
  } else {
    uint16_t* cp = static_cast<uint16_t*>(g.C) + m * g.ldc + n;
    if (g.beta != 0.f) val = fmaf(g.beta, bf2f(*cp), val);
    if (g.R) val += g.R[m * g.ldr + n];
    *cp = f2bf(val);
  }
}

template <bool AK, bool BK>
int launch_f32(const F32Args& g, int splits, hipStream_t s) {
  const int64_t tm = lz_cdiv(g.M, kTile), tn = lz_cdiv(g.N, kTile);
  LZ_REQUIRE(tm < 65536 && tn < (1ll << 31), "lz_gemm_f32: too many tiles (M %lld, N %lld)", (long long)g.M,
             (long long)g.N);
  dim3 grid((unsigned)tn, (unsigned)tm, (unsigned)splits);
  gemm_f32_kernel<AK, BK><<<grid, kThreads, 0, s>>>(g);
  return lz_check_launch("lz_gemm_f32");
}

int launch_layout(const F32Args& g, bool ak, bool bk, int splits, hipStream_t s) {
  if (ak && bk) return launch_f32<true, true>(g, splits, s);
  if (ak) return launch_f32<true, false>(g, splits, s);
  if (bk) return launch_f32<false, true>(g, splits, s);
  return launch_f32<false, false>(g, splits, s);
}

}  // namespace

// Workspace bytes lz_gemm_f32 uses for this shape (0 when K is not split).
LZ_EXPORT int64_t lz_gemm_f32_workspace(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return plan_workspace(make_plan(M, N, K), M, N);
}

// Number of K slices lz_gemm_f32 runs this shape in (1 = unsplit).
LZ_EXPORT int lz_gemm_f32_plan(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return make_plan(M, N, K).splits;
}

// fp32 operands, fp32 accumulation: C = alpha * sum_k A(m,k) B(n,k)
// (+ beta*C) (+ R), with the operand layouts of lz_gemm.  C: [M,N] fp32 or
// bf16 (ldc); R: optional fp32 [M,N] (ldr).  No alignment or size
// multiples are required; 16-byte aligned rows take 16-byte loads.  `ws`
// (ws_bytes long, may be null) holds the partial products when K is split;
// with less than lz_gemm_f32_workspace() bytes the product runs unsplit.
LZ_EXPORT int lz_gemm_f32(const float* A, int64_t lda, int a_kmajor, const float* B, int64_t ldb, int b_kmajor, void* C,
                          int64_t ldc, int c_dtype, const float* R, int64_t ldr, int64_t M, int64_t N, int64_t K,
                          float alpha, float beta, void* ws, int64_t ws_bytes, void* stream) {
  LZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "lz_gemm_f32: negative shape");
  if (M == 0 || N == 0) return LZ_OK;
  LZ_REQUIRE(C, "lz_gemm_f32: null output");
  LZ_REQUIRE(K == 0 || (A && B), "lz_gemm_f32: null operand");
  LZ_REQUIRE(c_dtype == LZ_F32 || c_dtype == LZ_BF16, "lz_gemm_f32: bad output dtype %d", c_dtype);
  LZ_REQUIRE(K == 0 || (lda >= (a_kmajor ? K : M) && ldb >= (b_kmajor ? K : N)), "lz_gemm_f32: bad operand stride");
  LZ_REQUIRE(ldc >= N && (R == nullptr || ldr >= N), "lz_gemm_f32: bad output stride");
  LZ_REQUIRE(ws_bytes >= 0 && (ws == nullptr || lz_aligned16(ws)), "lz_gemm_f32: workspace must be 16-byte aligned");
  F32Args g;
  g.A = A;
  g.B = B;
  g.C = C;
  g.R = R;
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
  g.a_vec = lz_aligned16(A) && lda % 4 == 0;
  g.b_vec = lz_aligned16(B) && ldb % 4 == 0;
  g.kper = K;
  g.slab = 0;
  hipStream_t s = lz_stream(stream);
  const bool ak = a_kmajor != 0, bk = b_kmajor != 0;
  const Plan p = make_plan(M, N, K);
  if (p.splits == 1 || ws == nullptr || ws_bytes < plan_workspace(p, M, N)) return launch_layout(g, ak, bk, 1, s);
  F32Args gs = g;  // partial products into fp32 slabs [splits][M][N]
  gs.C = ws;
  gs.kper = p.kper;
  gs.slab = M * N;
  int rc = launch_layout(gs, ak, bk, p.splits, s);
  if (rc) return rc;
  g.slab = M * N;
  splitk_reduce_f32_kernel<<<(unsigned)lz_cdiv(M * N, 256), 256, 0, s>>>(g, static_cast<const float*>(ws), p.splits);
  return lz_check_launch("lz_gemm_f32(split-K reduce)");
}
