// bf16 / fp16 GEMM on CDNA4 matrix cores:
//
//   C[M,N] = alpha * sum_k A(m,k) B(n,k)  (+ beta * C)  (+ R)
//
// Each operand is stored either K-major (A(m,k) = A[m*lda + k], the layout of
// nn.Linear's x . W^T, reference model/llama.py:81-84, 139-141, 178) or
// M/N-major (A(m,k) = A[k*lda + m]).  The three products of a linear layer
// map onto one kernel without transposing anything in HBM:
//   forward      y  = x  . W^T : A = x  K-major, B = W  K-major
//   input grad   dx = dy . W   : A = dy K-major, B = W  N-major
//   weight grad  dW = dy^T . x : A = dy M-major, B = x  N-major
// fp32 accumulation, bf16 or fp32 output, optional residual add (the block's
// `x + f(x)`, model/llama.py:158-159) and optional accumulation into an
// existing C (gradient accumulation).
//
// Tiling: a workgroup computes a BM x BN tile in 64-deep K steps staged
// through double-buffered LDS.  LDS always holds K-major rows padded to 144
// bytes, so the 16-byte fragment reads of 8 (or 16) consecutive lanes fall on
// distinct banks.  An M/N-major operand is loaded as 8x8 blocks (8 K rows of
// 8 contiguous elements) and transposed in registers before the LDS write.
// Each wave owns a (BM/WM) x (BN/WN) sub-tile of 32x32
// v_mfma_f32_32x32x16_bf16 tiles; the MFMA computes D = B_tile . A_tile^T so
// each lane ends up holding 4 consecutive output columns of one output row.
// Global loads for step k+1 are in flight while step k's MFMAs run.
// Workgroup ids are remapped so that consecutive tiles of one M-band land on
// the same XCD (its L2 then serves the shared operand rows).
#include <algorithm>
#include <cmath>
#include "lz_common.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// One 32x32x16 MFMA of the operand format F (FmtBF16 or FmtF16).  Fragments
// travel as bf16x8_t whatever the format: they are 16 raw bytes per lane.
template <typename F>
__device__ __forceinline__ f32x16_t mfma16(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
  if constexpr (F::kDtype == LZ_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// One 16x16x32 MFMA of the operand format F.  The direct-to-LDS kernels use
// this shape: on MI355X a stream of independent 16x16x32 MFMAs (128
// accumulator registers per wave, two waves per SIMD, as in these kernels)
// runs at about 2.39 GHz and 2.46 PFLOP/s, the same work as 32x32x16 MFMAs at
// about 2.14 GHz and 2.19 PFLOP/s: the same issue efficiency per clock, a
// higher clock under the power limit.  At the 256x256 tile, under sustained
// load, the forward product went from 1.23 to 1.31 PFLOP/s (O projection)
// and from 1.30 to 1.37 (gate|up); the gradient layouts, whose transposed
// LDS reads (ds_read_b64_tr_b16, about 150 bytes per clock per CU against
// about 220 for ds_read_b128) keep them near the LDS bound, by 1-2 %.
template <typename F>
__device__ __forceinline__ f32x4_t mfma_k32(const bf16x8_t& a, const bf16x8_t& b, const f32x4_t& c) {
  if constexpr (F::kDtype == LZ_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Accumulator fragments of an MI x MI MFMA tile (MI = 32: 32x32x16, 16 floats
// per lane; MI = 16: 16x16x32, 4 floats per lane).  The products are computed
// as D = B_tile . A_tile^T, so every lane holds groups of 4 consecutive output
// columns of one output row: group g (floats 4g..4g+3) of fragment (i, j) is
// row acc_row(i), columns acc_col(j, g) .. +3 of the wave's tile.
template <int MI>
struct Acc;
template <>
struct Acc<32> {
  typedef f32x16_t T;
  static constexpr int kGroups = 4;
};
template <>
struct Acc<16> {
  typedef f32x4_t T;
  static constexpr int kGroups = 1;
};
template <int MI>
__device__ __forceinline__ int acc_row(int i, int lane) {
  return i * MI + (lane & (MI - 1));
}
template <int MI>
__device__ __forceinline__ int acc_col(int j, int g, int lane) {
  return MI == 32 ? j * 32 + 8 * g + 4 * (lane >> 5) : j * 16 + 4 * (lane >> 4);
}

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
  int c_f32;      // output dtype fp32 (else the operands' 16-bit format)
  int vec_store;  // N, ldc, ldr multiples of 4 and pointers aligned
  int vec16;      // C rows (and R rows) start 16-byte aligned: row-contiguous 16-byte epilogue
  int r16;        // R rows 16-byte aligned too: the residual joins the 16-byte bf16 epilogue
  int64_t kper;   // K range of one split (multiple of 64); blockIdx.y is the split
  int64_t slab;   // elements between the fp32 partial slabs of consecutive splits
};

// Elementwise sum of two 8-value 16-bit pieces, rounded once.
template <typename F>
__device__ __forceinline__ uint4 add16x8(const uint4& a, const uint4& b) {
  const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    o[k] = F::pack2(F::to_f(aw[k] & 0xffff) + F::to_f(bw[k] & 0xffff), F::to_f(aw[k] >> 16) + F::to_f(bw[k] >> 16));
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// A 16-bit output with a residual is rounded twice, as the reference's
// separate ops are (the nn.Linear output in bf16, then x + y in bf16,
// model/llama.py:158-159): the product is rounded to the format before R is
// added and the sum is rounded on the store.  fp32 outputs add R unrounded.
template <typename F>
__device__ __forceinline__ float with_residual(float v, uint32_t r16) { return F::round(v) + F::to_f(r16 & 0xffff); }

template <typename F>
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
        o[0] += F::to_f(r.x & 0xffff); o[1] += F::to_f(r.x >> 16); o[2] += F::to_f(r.y & 0xffff); o[3] += F::to_f(r.y >> 16);
      }
      *cp = make_float4(o[0], o[1], o[2], o[3]);
    } else {
      uint2* cp = reinterpret_cast<uint2*>(static_cast<uint16_t*>(g.C) + m * g.ldc + n);
      if (g.beta != 0.f) {
        uint2 c = *cp;
        o[0] = fmaf(g.beta, F::to_f(c.x & 0xffff), o[0]); o[1] = fmaf(g.beta, F::to_f(c.x >> 16), o[1]);
        o[2] = fmaf(g.beta, F::to_f(c.y & 0xffff), o[2]); o[3] = fmaf(g.beta, F::to_f(c.y >> 16), o[3]);
      }
      if (g.R) {
        uint2 r = *reinterpret_cast<const uint2*>(g.R + m * g.ldr + n);
        o[0] = with_residual<F>(o[0], r.x & 0xffff); o[1] = with_residual<F>(o[1], r.x >> 16);
        o[2] = with_residual<F>(o[2], r.y & 0xffff); o[3] = with_residual<F>(o[3], r.y >> 16);
      }
      uint2 w;
      w.x = (uint32_t)F::from_f(o[0]) | ((uint32_t)F::from_f(o[1]) << 16);
      w.y = (uint32_t)F::from_f(o[2]) | ((uint32_t)F::from_f(o[3]) << 16);
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
      if (g.R) val += F::to_f(g.R[m * g.ldr + nn]);
      *cp = val;
    } else {
      uint16_t* cp = static_cast<uint16_t*>(g.C) + m * g.ldc + nn;
      if (g.beta != 0.f) val = fmaf(g.beta, F::to_f(*cp), val);
      if (g.R) val = with_residual<F>(val, g.R[m * g.ldr + nn]);
      *cp = F::from_f(val);
    }
  }
}

// Maps the linear workgroup id to a (tile_m, tile_n) pair.  Hardware places
// workgroup i on XCD i % 8; the remap gives each XCD a contiguous range of
// logical tiles, and the logical order walks groups of kGroupM M-tiles across
// all N-tiles so an XCD's concurrently running tiles share A rows and B rows.
__device__ __forceinline__ void tile_coords(int64_t pid, int64_t tiles_m, int64_t tiles_n, int64_t& tm, int64_t& tn) {
  constexpr int kXcd = 8, kGroupM = 4;
  const int64_t nblk = tiles_m * tiles_n;
  if (nblk % kXcd == 0) pid = (pid % kXcd) * (nblk / kXcd) + pid / kXcd;
  const int64_t per_group = (int64_t)kGroupM * tiles_n;
  const int64_t group = pid / per_group;
  const int64_t first_m = group * kGroupM;
  const int64_t gsize = min((int64_t)kGroupM, tiles_m - first_m);
  const int64_t in_group = pid - group * per_group;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

// One operand tile (ROWS rows of the M or N dimension x 64 K) moving from HBM
// through registers into a K-major LDS buffer.
template <int ROWS, int THREADS, bool KMAJOR>
struct TileLoader {
  // K-major: ROWS*8 chunks of 16 bytes (8 K values of one row).
  // M/N-major: ROWS 8x8 blocks (8 K rows x 8 contiguous M/N values).
  static constexpr int kUnits = ROWS * 8 / (KMAJOR ? 1 : 8);
  static constexpr int kPer = (kUnits + THREADS - 1) / THREADS;
  static constexpr int kRegs = KMAJOR ? kPer : kPer * 8;
  static constexpr bool kFull = kUnits % THREADS == 0;
  uint4 r[kRegs];

  // CHECK=false: the whole tile (rows and 64 K) is in range.  CHECK=true:
  // addresses are clamped into the operand and out-of-range data is zeroed
  // with a mask, so no load sits behind a branch.
  template <bool CHECK>
  __device__ __forceinline__ void load(const uint16_t* __restrict__ p, int64_t ld, int64_t row0, int64_t nrows,
                                       int64_t k0, int64_t kend, int tid) {
    if constexpr (KMAJOR) {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int c = tid + i * THREADS;
        const int row = c >> 3, ch = c & 7;
        const int64_t gr = row0 + row, gk = k0 + ch * 8;
        if constexpr (!CHECK) {
          r[i] = *reinterpret_cast<const uint4*>(p + gr * ld + gk);
        } else {
          const uint32_t msk = ((kFull || c < kUnits) && gr < nrows && gk < kend) ? ~0u : 0u;
          const uint4 v = *reinterpret_cast<const uint4*>(p + min(gr, nrows - 1) * ld + min(gk, kend - 8));
          r[i] = make_uint4(v.x & msk, v.y & msk, v.z & msk, v.w & msk);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int b = tid + i * THREADS;
        const int kb = b & 7, rb = b >> 3;  // 8 consecutive lanes: 8 K blocks of one row block
        const int64_t gr = row0 + rb * 8;
        if constexpr (!CHECK) {
          const int64_t rr = (kFull || b < kUnits) ? gr : row0;
#pragma unroll
          for (int j = 0; j < 8; ++j) r[i * 8 + j] = *reinterpret_cast<const uint4*>(p + (k0 + kb * 8 + j) * ld + rr);
        } else {
          const bool ok = (kFull || b < kUnits) && gr < nrows;
          const int64_t grc = min(gr, nrows - 8);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int64_t gk = k0 + kb * 8 + j;
            const uint32_t msk = (ok && gk < kend) ? ~0u : 0u;
            const uint4 v = *reinterpret_cast<const uint4*>(p + min(gk, kend - 1) * ld + grc);
            r[i * 8 + j] = make_uint4(v.x & msk, v.y & msk, v.z & msk, v.w & msk);
          }
        }
      }
    }
  }

  __device__ __forceinline__ void store(char* lds, int tid) {
    if constexpr (KMAJOR) {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int c = tid + i * THREADS;
        if (kFull || c < kUnits) *reinterpret_cast<uint4*>(lds + (c >> 3) * kRowBytes + (c & 7) * 16) = r[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int b = tid + i * THREADS;
        if (!kFull && b >= kUnits) continue;
        const int kb = b & 7, rb = b >> 3;
        // r[i*8 + j] holds K row j, elements e = 0..7 as dwords (e=2q, 2q+1);
        // output row e needs K = 0..7 of element e.
        const uint32_t* x = reinterpret_cast<const uint32_t*>(&r[i * 8]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int q = e >> 1;
          uint32_t w[4];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const uint32_t lo = x[(2 * jj) * 4 + q], hi = x[(2 * jj + 1) * 4 + q];
            w[jj] = (e & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
          }
          *reinterpret_cast<uint4*>(lds + (rb * 8 + e) * kRowBytes + kb * 16) = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
    }
  }
};

// Chunk swizzle of a staged epilogue row of kRow bytes: rows that share a
// 256-byte bank window are told apart by the XOR, so 16 lanes writing one
// chunk of 16 consecutive rows (or reading 16 chunks of a row) hit 16
// distinct 16-byte bank groups.
template <int kRow>
__device__ __forceinline__ int epi_swz(int row) {
  constexpr int kPer256 = kRow >= 256 ? 1 : 256 / kRow;
  constexpr int kMask = (kRow / 16 - 1) < 15 ? (kRow / 16 - 1) : 15;
  return (row / kPer256) & kMask;
}

// Staged epilogue rows of kRow bytes: a power-of-two number of 16-byte chunks
// is XOR-swizzled in place (epi_swz); other widths (the 48-wide wave tiles of
// 192-wide tiles: 6 bf16 or 12 fp32 chunks) are padded by one chunk instead,
// an odd pitch in chunks that staggers consecutive rows over the bank groups.
template <int kRow>
constexpr bool epi_pow2() {
  return ((kRow / 16) & (kRow / 16 - 1)) == 0;
}
template <int kRow>
constexpr int epi_pitch() {
  return epi_pow2<kRow>() ? kRow : kRow + 16;
}
template <int kRow>
__device__ __forceinline__ int epi_off(int row, int chunk) {
  if constexpr (epi_pow2<kRow>()) return row * kRow + ((chunk ^ epi_swz<kRow>(row)) << 4);
  else return row * epi_pitch<kRow>() + (chunk << 4);
}
// LDS bytes one wave's region of store_tile16 takes: TM bf16 rows or TM/2 fp32
// rows of TN values.
template <int TM, int TN>
constexpr int epi_wave_bytes() {
  return TM * epi_pitch<TN * 2>() > (TM / 2) * epi_pitch<TN * 4>() ? TM * epi_pitch<TN * 2>()
                                                                    : (TM / 2) * epi_pitch<TN * 4>();
}

// Interior tiles, 16-byte path: each wave parks its TM x TN sub-tile in a
// private LDS region (rows of TN values, 16-byte chunks XOR-swizzled so that
// both the accumulator-layout writes and the row-wise reads are free of bank
// conflicts), then writes whole 16-byte pieces of consecutive row bytes, so a
// store instruction covers full cache lines.  fp32 output goes in two passes
// of TM/2 rows.  Needs WM*WN*epi_wave_bytes<TM, TN>() bytes of LDS (BM*BN*2
// for power-of-two wave tile widths).
// Parks a wave's TM x TN accumulator tile in its LDS region as 16-bit values
// (scaled by alpha, rounded once): rows of TN values (kRow = 2*TN bytes),
// 16-byte chunks XOR-swizzled by epi_swz, so that the accumulator-layout
// writes and the row-wise reads are free of bank conflicts.
template <typename F, int MI, int FM, int FN, int kRow>
__device__ __forceinline__ void park16(const typename Acc<MI>::T (&acc)[FM][FN], char* st, int lane, float alpha) {
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int q = 0; q < Acc<MI>::kGroups; ++q) {
        const int row = acc_row<MI>(i, lane), byte = 2 * acc_col<MI>(j, q, lane);
        *reinterpret_cast<uint2*>(st + epi_off<kRow>(row, byte >> 4) + (byte & 15)) =
            make_uint2(F::pack2(acc[i][j][4 * q] * alpha, acc[i][j][4 * q + 1] * alpha),
                       F::pack2(acc[i][j][4 * q + 2] * alpha, acc[i][j][4 * q + 3] * alpha));
      }
}

template <typename F, int MI, int BM, int BN, int WM, int WN>
__device__ __forceinline__ void store_tile16(const GemmArgs& go, typename Acc<MI>::T (&acc)[BM / WM / MI][BN / WN / MI],
                                             int64_t m0, int64_t n0, char* smem, int lane, int wave) {
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / MI, FN = TN / MI;
  static_assert(FM % 2 == 0, "fp32 output is staged in two halves");
  const int wm = wave / WN, wn = wave % WN;
  const int64_t mrow0 = m0 + wm * TM, ncol0 = n0 + wn * TN;
  char* st = smem + wave * epi_wave_bytes<TM, TN>();
  if (!go.c_f32) {
    constexpr int kRow = TN * 2, kChunks = kRow / 16;  // bytes and 16-byte chunks per row
    static_assert(kChunks >= 4 && kChunks <= 64, "bf16 rows of 32 to 512 values");
    // beta == 0: stage bf16 values (the product rounded once) and store whole
    // 16-byte row pieces; a residual is added to each piece on the way out
    const bool plain = go.beta == 0.f && (go.R == nullptr || go.r16);
    if (plain) {
      park16<F, MI, FM, FN, kRow>(acc, st, lane, go.alpha);
      asm volatile("" ::: "memory");
      constexpr int kIters = TM * kChunks / 64;
      if (go.R == nullptr) {
        // 64 lanes x 16 bytes per store: whole rows (or 64-chunk row pieces)
#pragma unroll
        for (int t = 0; t < kIters; ++t) {
          const int idx = t * 64 + lane, row = idx / kChunks, chunk = idx % kChunks;
          const uint4 v = *reinterpret_cast<const uint4*>(st + epi_off<kRow>(row, chunk));
          st_nt16(static_cast<uint16_t*>(go.C) + (mrow0 + row) * go.ldc + ncol0 + chunk * 8, v);
        }
        return;
      }
      // with the residual: the R pieces of 8 stores are loaded together (R may
      // alias the output, so the compiler would not hoist them past the stores)
      constexpr int kBlk = kIters < 8 ? kIters : kIters % 8 == 0 ? 8 : kIters % 6 == 0 ? 6 : 4;
      static_assert(kIters % kBlk == 0, "store blocks must tile the wave's rows");
#pragma unroll
      for (int t0 = 0; t0 < kIters; t0 += kBlk) {
        uint4 rv[kBlk];
#pragma unroll
        for (int u = 0; u < kBlk; ++u) {
          const int idx = (t0 + u) * 64 + lane, row = idx / kChunks, chunk = idx % kChunks;
          rv[u] = *reinterpret_cast<const uint4*>(go.R + (mrow0 + row) * go.ldr + ncol0 + chunk * 8);
        }
#pragma unroll
        for (int u = 0; u < kBlk; ++u) {
          const int idx = (t0 + u) * 64 + lane, row = idx / kChunks, chunk = idx % kChunks;
          const uint4 v = *reinterpret_cast<const uint4*>(st + epi_off<kRow>(row, chunk));
          st_nt16(static_cast<uint16_t*>(go.C) + (mrow0 + row) * go.ldc + ncol0 + chunk * 8, add16x8<F>(v, rv[u]));
        }
      }
      return;
    }
  }
  // fp32 values staged (fp32 output, or bf16 output with beta / residual,
  // which are applied before the single rounding): two passes of TM/2 rows.
  // The stores go in blocks of kBlk: each block first issues all of its loads
  // of C (beta) and R, so that they are in flight together instead of one
  // load-use round trip per store (C and R may alias the output, so the
  // compiler cannot hoist them past the stores itself).
  constexpr int kRow = TN * 4, kChunks = kRow / 16;
  constexpr int kIters = (TM / 2) * kChunks / 64, kBlk = kIters < 4 ? kIters : 4;
  static_assert(kChunks >= 4 && kChunks <= 64, "fp32 rows of 16 to 256 values");
  static_assert(kIters % kBlk == 0, "store blocks must tile a pass");
  const bool has_c = go.beta != 0.f, has_r = go.R != nullptr;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
#pragma unroll
    for (int ii = 0; ii < FM / 2; ++ii) {
      const int i = p * (FM / 2) + ii;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < Acc<MI>::kGroups; ++q) {
          const int row = acc_row<MI>(ii, lane), chunk = acc_col<MI>(j, q, lane) >> 2;
          *reinterpret_cast<float4*>(st + epi_off<kRow>(row, chunk)) =
              make_float4(acc[i][j][4 * q] * go.alpha, acc[i][j][4 * q + 1] * go.alpha,
                          acc[i][j][4 * q + 2] * go.alpha, acc[i][j][4 * q + 3] * go.alpha);
        }
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int t0 = 0; t0 < kIters; t0 += kBlk) {
      uint4 cpre[kBlk];  // beta's C: fp32 x4, or bf16 x4 in .x/.y
      uint2 rpre[kBlk];  // residual, bf16 x4
#pragma unroll
      for (int u = 0; u < kBlk; ++u) {
        const int idx = (t0 + u) * 64 + lane, row = idx / kChunks, chunk = idx % kChunks;
        const int64_t m = mrow0 + p * (TM / 2) + row, n = ncol0 + chunk * 4;
        cpre[u] = make_uint4(0u, 0u, 0u, 0u);
        rpre[u] = make_uint2(0u, 0u);
        if (has_c) {
          if (go.c_f32) {
            cpre[u] = *reinterpret_cast<const uint4*>(static_cast<const float*>(go.C) + m * go.ldc + n);
          } else {
            const uint2 c = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(go.C) + m * go.ldc + n);
            cpre[u].x = c.x;
            cpre[u].y = c.y;
          }
        }
        if (has_r) rpre[u] = *reinterpret_cast<const uint2*>(go.R + m * go.ldr + n);
      }
#pragma unroll
      for (int u = 0; u < kBlk; ++u) {
        const int idx = (t0 + u) * 64 + lane, row = idx / kChunks, chunk = idx % kChunks;
        const uint4 v = *reinterpret_cast<const uint4*>(st + epi_off<kRow>(row, chunk));
        const int64_t m = mrow0 + p * (TM / 2) + row, n = ncol0 + chunk * 4;
        float o[4] = {__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w)};
        if (has_c) {
          const uint4 c = cpre[u];
          if (go.c_f32) {
            o[0] = fmaf(go.beta, __uint_as_float(c.x), o[0]); o[1] = fmaf(go.beta, __uint_as_float(c.y), o[1]);
            o[2] = fmaf(go.beta, __uint_as_float(c.z), o[2]); o[3] = fmaf(go.beta, __uint_as_float(c.w), o[3]);
          } else {
            o[0] = fmaf(go.beta, F::to_f(c.x & 0xffff), o[0]); o[1] = fmaf(go.beta, F::to_f(c.x >> 16), o[1]);
            o[2] = fmaf(go.beta, F::to_f(c.y & 0xffff), o[2]); o[3] = fmaf(go.beta, F::to_f(c.y >> 16), o[3]);
          }
        }
        if (has_r) {
          const uint2 r = rpre[u];
          if (go.c_f32) {
            o[0] += F::to_f(r.x & 0xffff); o[1] += F::to_f(r.x >> 16); o[2] += F::to_f(r.y & 0xffff); o[3] += F::to_f(r.y >> 16);
          } else {
            o[0] = with_residual<F>(o[0], r.x & 0xffff); o[1] = with_residual<F>(o[1], r.x >> 16);
            o[2] = with_residual<F>(o[2], r.y & 0xffff); o[3] = with_residual<F>(o[3], r.y >> 16);
          }
        }
        if (go.c_f32) {
          st_nt16(static_cast<float*>(go.C) + m * go.ldc + n, make_uint4(
              __float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]), __float_as_uint(o[3])));
        } else {
          *reinterpret_cast<uint2*>(static_cast<uint16_t*>(go.C) + m * go.ldc + n) =
              make_uint2(F::pack2(o[0], o[1]), F::pack2(o[2], o[3]));
        }
      }
    }
    asm volatile("" ::: "memory");
  }
}

// Writes a workgroup's BM x BN accumulator tile (layout: Acc<MI>).
// Interior tiles with 16-byte aligned rows and wave tiles up to 64 wide take
// store_tile16; other interior tiles store each lane's 4-column groups
// straight from the accumulators (8 or 16 bytes) with the row address formed
// once per fragment row band; edge tiles go through LDS one MI-row band at a
// time and are written as whole rows with bounds checks, so the accumulators
// are never indexed dynamically.  `smem` must be free and at least
// max(WM*WN*MI*(BN/WN+4)*4, BM*BN*2) bytes.
template <typename F, int MI, int BM, int BN, int WM, int WN>
__device__ __forceinline__ void store_tile(const GemmArgs& go, typename Acc<MI>::T (&acc)[BM / WM / MI][BN / WN / MI],
                                           int64_t m0, int64_t n0, char* smem, int lane, int wave) {
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / MI, FN = TN / MI, G = Acc<MI>::kGroups;
  const int wm = wave / WN, wn = wave % WN;
  if constexpr (TN <= 64) {  // (wider wave tiles run out of registers in the staged path)
    if (m0 + BM <= go.M && n0 + BN <= go.N && go.vec16) {
      store_tile16<F, MI, BM, BN, WM, WN>(go, acc, m0, n0, smem, lane, wave);
      return;
    }
  }
  if (m0 + BM <= go.M && n0 + BN <= go.N && go.vec_store) {
    const int64_t ncol0 = n0 + wn * TN;
    if (go.c_f32) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int64_t m = m0 + wm * TM + acc_row<MI>(i, lane);
        float* crow = static_cast<float*>(go.C) + m * go.ldc + ncol0;
        const uint16_t* rrow = go.R ? go.R + m * go.ldr + ncol0 : nullptr;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int q = 0; q < G; ++q) {
            const int c = acc_col<MI>(j, q, lane);
            float4 o = make_float4(acc[i][j][4 * q] * go.alpha, acc[i][j][4 * q + 1] * go.alpha,
                                   acc[i][j][4 * q + 2] * go.alpha, acc[i][j][4 * q + 3] * go.alpha);
            float4* cp = reinterpret_cast<float4*>(crow + c);
            if (go.beta != 0.f) {
              const float4 cv = *cp;
              o.x = fmaf(go.beta, cv.x, o.x); o.y = fmaf(go.beta, cv.y, o.y);
              o.z = fmaf(go.beta, cv.z, o.z); o.w = fmaf(go.beta, cv.w, o.w);
            }
            if (rrow) {
              const uint2 r = *reinterpret_cast<const uint2*>(rrow + c);
              o.x += F::to_f(r.x & 0xffff); o.y += F::to_f(r.x >> 16); o.z += F::to_f(r.y & 0xffff); o.w += F::to_f(r.y >> 16);
            }
            *cp = o;
          }
      }
    } else {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int64_t m = m0 + wm * TM + acc_row<MI>(i, lane);
        uint16_t* crow = static_cast<uint16_t*>(go.C) + m * go.ldc + ncol0;
        const uint16_t* rrow = go.R ? go.R + m * go.ldr + ncol0 : nullptr;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int q = 0; q < G; ++q) {
            const int c = acc_col<MI>(j, q, lane);
            float o[4] = {acc[i][j][4 * q] * go.alpha, acc[i][j][4 * q + 1] * go.alpha,
                          acc[i][j][4 * q + 2] * go.alpha, acc[i][j][4 * q + 3] * go.alpha};
            uint2* cp = reinterpret_cast<uint2*>(crow + c);
            if (go.beta != 0.f) {
              const uint2 cv = *cp;
              o[0] = fmaf(go.beta, F::to_f(cv.x & 0xffff), o[0]); o[1] = fmaf(go.beta, F::to_f(cv.x >> 16), o[1]);
              o[2] = fmaf(go.beta, F::to_f(cv.y & 0xffff), o[2]); o[3] = fmaf(go.beta, F::to_f(cv.y >> 16), o[3]);
            }
            if (rrow) {
              const uint2 r = *reinterpret_cast<const uint2*>(rrow + c);
              o[0] = with_residual<F>(o[0], r.x & 0xffff); o[1] = with_residual<F>(o[1], r.x >> 16);
              o[2] = with_residual<F>(o[2], r.y & 0xffff); o[3] = with_residual<F>(o[3], r.y >> 16);
            }
            *cp = make_uint2(F::pack2(o[0], o[1]), F::pack2(o[2], o[3]));
          }
      }
    }
    return;
  }
  constexpr int kPitch = TN + 4;  // floats; 16-byte aligned, staggers the banks of consecutive rows
  float* stage = reinterpret_cast<float*>(smem) + wave * MI * kPitch;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int q = 0; q < G; ++q)
        *reinterpret_cast<float4*>(stage + acc_row<MI>(0, lane) * kPitch + acc_col<MI>(j, q, lane)) =
            make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
    __syncthreads();
    const int64_t mband = m0 + wm * TM + i * MI, nband = n0 + wn * TN;
    for (int it = lane; it < MI * (TN / 4); it += 64) {
      const int r = it / (TN / 4), c4 = it % (TN / 4);
      const int64_t m = mband + r, n = nband + c4 * 4;
      if (m < go.M && n < go.N) {
        const float4 v4 = *reinterpret_cast<const float4*>(stage + r * kPitch + c4 * 4);
        const float v[4] = {v4.x, v4.y, v4.z, v4.w};
        store_out4<F>(go, m, n, v);
      }
    }
    __syncthreads();
  }
}

// Register-staged kernel: any operand layouts.  Global loads for K step k+1
// are in flight in registers while step k's MFMAs run, then written to the
// other LDS buffer (transposed on the way for an M/N-major operand).
template <typename F, int BM, int BN, int WM, int WN, bool AK, bool BK>
__global__ void __launch_bounds__(64 * WM * WN) gemm_kernel(GemmArgs g) {
  constexpr int kThreads = 64 * WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;  // wave sub-tile
  constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 MFMA tiles per wave
  constexpr int kStageBytes = (BM + BN) * kRowBytes;
  static_assert(WM * WN * 32 * (TN + 4) * 4 <= 2 * kStageBytes, "epilogue staging does not fit");

  __shared__ __attribute__((aligned(16))) char smem[2 * kStageBytes];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t tiles_m = lz_cdiv(g.M, BM), tiles_n = lz_cdiv(g.N, BN);
  int64_t tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = tm * BM, n0 = tn * BN;
  const int64_t kbeg = (int64_t)blockIdx.y * g.kper, kend = min(g.K, kbeg + g.kper);
  const int64_t ktiles = kend > kbeg ? lz_cdiv(kend - kbeg, kBK) : 0;
  // uniform per workgroup: the whole tile lies inside the operands
  const bool interior = m0 + BM <= g.M && n0 + BN <= g.N && (kend - kbeg) % kBK == 0;

  TileLoader<BM, kThreads, AK> la;
  TileLoader<BN, kThreads, BK> lb;
  auto gload = [&](int64_t k0) {
    if (interior) {
      la.template load<false>(g.A, g.lda, m0, g.M, k0, kend, tid);
      lb.template load<false>(g.B, g.ldb, n0, g.N, k0, kend, tid);
    } else {
      la.template load<true>(g.A, g.lda, m0, g.M, k0, kend, tid);
      lb.template load<true>(g.B, g.ldb, n0, g.N, k0, kend, tid);
    }
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  if (ktiles > 0) {
    gload(kbeg);
    la.store(smem, tid);
    lb.store(smem + BM * kRowBytes, tid);
  }
  __syncthreads();

  const int frag_row = lane & 31;
  const int frag_k = (lane >> 5) * 16;  // byte offset of this lane's 8 K values
  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < ktiles) gload(kbeg + (kt + 1) * kBK);
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
        for (int j = 0; j < FN; ++j)
          acc[i][j] = mfma16<F>(fa[j], fb[i], acc[i][j]);
    }
    if (kt + 1 < ktiles) {
      char* nxt = smem + (cur ^ 1) * kStageBytes;
      la.store(nxt, tid);
      lb.store(nxt + BM * kRowBytes, tid);
    }
    __syncthreads();
  }

  GemmArgs go = g;  // split-K: this split's fp32 slab
  if (g.slab) go.C = static_cast<float*>(g.C) + (int64_t)blockIdx.y * g.slab;
  store_tile<F, 32, BM, BN, WM, WN>(go, acc, m0, n0, smem, lane, wave);
}

// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// Direct-to-LDS kernel.
//
// Global data goes straight into LDS with global_load_lds_dwordx4 (each lane's
// 16 bytes land at the wave-uniform destination + 16*lane), so staging takes
// no registers and no LDS-write instructions.  K advances 64 per stage over two
// LDS stages: the loads for stage k+1 are issued right after the barrier that
// opens stage k (whose fence waits for stage k's loads).  Stages are stored as
// they lie in memory (K-major rows or M/N-major rows, unpadded, XOR-swizzled);
// an M/N-major operand's fragments come from ds_read_b64_tr_b16, which
// transposes 4x4 blocks of 16-bit values across each 16-lane group.  Rows
// (K-major) or columns (M/N-major) past M or N are clamped to valid memory;
// they only feed outputs that are not stored.
// ---------------------------------------------------------------------------
// LDS row swizzle: chunk c (8 K values) of row r sits in slot c ^ swz(r).
// For 4-chunk (64-byte) and 8-chunk (128-byte) rows this keeps the 16-byte
// reads of 8 or 16 consecutive rows on distinct banks.
template <int kChunks>
__device__ __forceinline__ int swz(int r) {
  if constexpr (kChunks == 4) return ((r >> 1) ^ (r >> 3)) & 3;
  else return ((r >> 1) ^ ((r & 1) << 2)) & 7;
}

// Swizzle of the 16-byte chunks of an M/N-major stage row (64 K rows of 256
// M/N values, 512 bytes): keeps each half-wave of ds_read_b64_tr_b16 (4
// consecutive rows x 64 bytes) on distinct banks.
__device__ __forceinline__ int swz_mn(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t* lds_v4i16_ptr;

// Swizzle of the 16-byte chunks of an M/N-major stage row of 192 M/N values
// (384 bytes, 24 chunks; consecutive rows start 128 bytes apart modulo the
// 256-byte bank window, so even and odd rows use opposite halves of it): an
// even XOR below 8 keeps chunk pairs together and inside their row, and gives
// the 8 rows r = 8G + 4rd + j (G = 0, 1; j = 0..3) that one half-wave of
// ds_read_b64_tr_b16 reads distinct 32-byte bank groups.
__device__ __forceinline__ int swz_mn192(int r) { return 2 * (((r >> 1) & 1) | (((r >> 3) & 1) << 1)); }

// Swizzle of the 16-byte chunks of a K-major stage row of 32 K (64 bytes,
// 4 chunks): the 16 lanes of a ds_read_b128 quarter-wave (16 consecutive rows,
// one logical chunk) land on 16 distinct 16-byte bank groups.
__device__ __forceinline__ int swz_k4(int r) { return (r >> 2) & 3; }

// One operand of the direct-to-LDS kernel: a 256 (M or N) x DBK (K) stage,
// 512 * DBK bytes, filled by wave loads of 1 KB (64 lanes x 16 bytes).
//   K-major: 256 rows of DBK K values (2*DBK bytes: 8 chunks swizzled by
//            swz<8> for DBK 64, 4 chunks swizzled by swz_k4 for DBK 32);
//            fragments are plain 16-byte reads.
//   M/N-major: DBK rows of kCols M/N values (256: 512 bytes, 32 chunks,
//            swizzled by swz_mn; 192: 384 bytes, 24 chunks, swizzled by
//            swz_mn192); fragments are two ds_read_b64_tr_b16 each.
// A K-major stage of kCols rows is the same code with fewer wave loads.
template <bool KMAJOR, int kPerWave, int DBK, int kCols = 256>
struct DmaOperand {
  static_assert(kCols == 256 || kCols == 192, "stages of 256 or 192 M/N values");
  static constexpr int kChunksK = DBK / 8;        // 16-byte chunks per K-major row
  static constexpr int kRowsK = 64 / kChunksK;    // K-major rows per wave load
  // Raw buffer starting at the tile's origin (row0, kbeg): the loads are
  // buffer_load ... lds with a 32-bit per-lane offset and the K step in the
  // scalar offset, which measured 3-9 % faster than 64-bit per-lane
  // addresses.  The host keeps every offset below 2^31 (dma_spans_fit).
  lz_v4i rsrc;
  uint32_t voff[kPerWave];  // per-lane byte offsets
  uint32_t kadv;            // bytes to advance per DBK-deep K step

  // pair > 0 (K-major only): tile rows 0-127 are rows row0.. and tile rows
  // 128-255 are rows pair+row0.. of the operand (two 128-row halves taken
  // `pair` rows apart, e.g. matching gate and up rows of a fused weight).
  __device__ __forceinline__ void init(const uint16_t* p, int64_t ld, int64_t row0, int64_t nrows, int64_t kbeg,
                                       int wave, int lane, int64_t pair = 0) {
    const uint16_t* base = KMAJOR ? p + row0 * ld + kbeg : p + kbeg * ld + row0;
    rsrc = lz_buffer_rsrc(base);
#pragma unroll
    for (int q = 0; q < kPerWave; ++q) {
      if constexpr (KMAJOR) {
        const int r = (wave * kPerWave + q) * kRowsK + lane / kChunksK;
        const int c = (lane % kChunksK) ^ (DBK == 64 ? swz<8>(r) : swz_k4(r));
        const int64_t gr = pair > 0 ? (r & 127) + (r >> 7) * pair : min(row0 + r, nrows - 1) - row0;
        voff[q] = (uint32_t)((gr * ld + c * 8) * 2);
      } else if constexpr (kCols == 192) {
        // a wave load's 1 KB spans 2 2/3 rows: the row and the chunk slot
        // follow from the 16-byte slot's position in the stage
        const int pos = (wave * kPerWave + q) * 64 + lane;
        const int r = pos / 24, c = (pos % 24) ^ swz_mn192(r);
        voff[q] = (uint32_t)((r * ld + (min(row0 + c * 8, nrows - 8) - row0)) * 2);
      } else {
        const int r = (wave * kPerWave + q) * 2 + (lane >> 5);
        const int c = (lane & 31) ^ swz_mn(r);
        voff[q] = (uint32_t)((r * ld + (min(row0 + c * 8, nrows - 8) - row0)) * 2);
      }
    }
    kadv = (uint32_t)((KMAJOR ? DBK : DBK * ld) * 2);
  }

  __device__ __forceinline__ void issue(char* dst, int wave, int kt) const {
#pragma unroll
    for (int q = 0; q < kPerWave; ++q)
      lz_dma16(rsrc, voff[q], (uint32_t)kt * kadv, dst + (wave * kPerWave + q) * 1024);
  }
};

// Per-lane LDS offsets of this wave's NF 16-row fragments (16-row blocks
// blk0 .. blk0+NF-1 of the operand) for the two 32-deep K slices of a 64-deep
// stage, in the operand layout of the 16x16x32 MFMA: lane l supplies row
// l % 16 of the fragment and K values 8*(l/16) .. +7 of the slice.
template <bool KMAJOR, int NF, int kCols = 256>
struct DmaFrags {
  static constexpr int kRowBytes = kCols * 2;  // M/N-major stage row
  int kb[KMAJOR ? 2 : 1];              // K-major
  int base[2], ioff[KMAJOR ? 1 : NF];  // M/N-major

  __device__ __forceinline__ void init(int blk0, int lane) {
    if constexpr (KMAJOR) {
      // a K-major stage row is 64 K (8 chunks of 8, swizzled by swz<8>); chunk
      // 4*kk + l/16 of row r = 16*(blk0 + f) + l%16.  swz<8>(r) depends only
      // on r % 16, so fragment f sits at a constant offset f*16*128 from
      // fragment 0 (two offset registers per operand, not two per fragment).
      // 8 consecutive lanes read 8 rows of one logical chunk: distinct banks
      // under swz<8>.
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int r = blk0 * 16 + (lane & 15);
        kb[kk] = r * 128 + (((4 * kk + (lane >> 4)) ^ swz<8>(r)) << 4);
      }
    } else if constexpr (kCols == 192) {
      // The same reads on 384-byte rows: row r = 32*kk + 8G + 4*rd + j has
      // swz_mn192(r) = 2*((j >> 1) | ((G % 2) << 1)) for either rd, an even
      // value, so chunk (2*blk + q/2) ^ swz sits at slot (2*blk ^ swz) + q/2.
      const int p = lane & 15, grp = lane >> 4, j = p >> 2, q = p & 3;
      const int t = 2 * ((j >> 1) | ((grp & 1) << 1));
#pragma unroll
      for (int rd = 0; rd < 2; ++rd) base[rd] = (8 * grp + 4 * rd + j) * kRowBytes + ((q >> 1) << 4) + (q & 1) * 8;
#pragma unroll
      for (int f = 0; f < NF; ++f) ioff[f] = ((2 * (blk0 + f)) ^ t) << 4;
    } else {
      // An M/N-major stage holds 64 K rows of 256 M/N values (512 bytes, 32
      // chunks swizzled by swz_mn).  ds_read_b64_tr_b16 lets the 16 lanes of
      // group G = l/16 load a 4 (K) x 16 (M/N) block, lane p = 4j + q reading
      // K row j, columns 4q .. 4q+3, and gives lane p column p at the 4 K
      // rows.  Two reads per fragment cover K rows 32*kk + 8G + 4*rd + 0..3
      // (rd = 0, 1) of column block blk: lane p then holds column 16*blk + p
      // at K 8G .. 8G+7 of the slice, the MFMA's operand layout.
      //   chunk of (row r, column 16*blk + 4q) = (2*blk + q/2) ^ swz_mn(r),
      //   swz_mn(r) = 4j + 2*(G%2) + rd for these rows, so the chunk splits
      //   into (2*blk ^ (4j + 2*(G%2))) (per fragment: ioff) and (q/2 ^ rd)
      //   (per read: base).  Each group's 8 chunks of 4 rows hit distinct
      //   16-byte bank groups, as do the two groups of a half-wave.
      const int p = lane & 15, grp = lane >> 4, j = p >> 2, q = p & 3;
#pragma unroll
      for (int rd = 0; rd < 2; ++rd)
        base[rd] = (8 * grp + 4 * rd + j) * 512 + (((q >> 1) ^ rd) << 4) + (q & 1) * 8;
#pragma unroll
      for (int f = 0; f < NF; ++f) ioff[f] = ((2 * (blk0 + f)) ^ (4 * j + 2 * (grp & 1))) << 4;
    }
  }

  __device__ __forceinline__ bf16x8_t frag(const char* op, int f, int kk) const {
    if constexpr (KMAJOR) {
      return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(op + f * 16 * 128 + kb[kk]));
    } else {
      const char* blk = op + kk * 32 * kRowBytes + ioff[f];
      const v4i16_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(blk + base[0]));
      const v4i16_t y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(blk + base[1]));
      const uint2 xw = __builtin_bit_cast(uint2, x), yw = __builtin_bit_cast(uint2, y);
      return __builtin_bit_cast(bf16x8_t, make_uint4(xw.x, xw.y, yw.x, yw.y));
    }
  }
};

// Fragments of one 32-deep K slice: fa (B operand, FN of them) and fb (A
// operand, FM), read from the LDS stage at (sa, sb).
template <bool AK, bool BK, int FM, int FN, int kColsB>
__device__ __forceinline__ void dma_load_frags(const DmaFrags<AK, FM>& fra, const DmaFrags<BK, FN, kColsB>& frb, const char* sa,
                                               const char* sb, int kk, bf16x8_t (&fa)[FN], bf16x8_t (&fb)[FM]) {
#pragma unroll
  for (int j = 0; j < FN; ++j) fa[j] = frb.frag(sb, j, kk);
#pragma unroll
  for (int i = 0; i < FM; ++i) fb[i] = fra.frag(sa, i, kk);
}

template <typename F, int FM, int FN>
__device__ __forceinline__ void dma_mfma(f32x4_t (&acc)[FM][FN], const bf16x8_t (&fa)[FN], const bf16x8_t (&fb)[FM]) {
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = mfma_k32<F>(fa[j], fb[i], acc[i][j]);
}

// Scheduling of one K slice: NM MFMAs, each followed by up to ceil(R/NM) of
// the R LDS reads of the next slice (instruction-group barriers: 0x008 =
// MFMA, 0x100 = LDS read).
template <int R, int NM, int Q = 0>
__device__ __forceinline__ void sched_slice() {
  if constexpr (Q < NM) {
    constexpr int rpm = (R + NM - 1) / NM;
    constexpr int left = R - Q * rpm;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if constexpr (left > 0) __builtin_amdgcn_sched_group_barrier(0x100, left < rpm ? left : rpm, 0);
    sched_slice<R, NM, Q + 1>();
  }
}


// Direct-to-LDS kernel, any operand layouts: 256x256 tile, 64-deep K steps
// over two LDS stages of 2 x 512 x 64 bytes; 8 waves of 128x64, each an 8x4
// grid of 16x16x32 MFMA tiles (two 32-deep slices per stage).  K must be a
// multiple of 64 in every split; an M-major A needs M % 8 == 0 (N-major B:
// N % 8 == 0).
//
// Schedule (the mid-step barrier): half of the waves (one per SIMD) issue all
// stage loads, so the other wave on each SIMD keeps issuing MFMAs while the
// loads queue, and the barrier sits in the middle of a step, after the last
// LDS reads of the current stage, so that the MFMAs of its second slice run
// while the next stage's first fragments are read.  Measured on the 1B step's
// shapes against the plain step (all waves load, barrier at the step's
// start): input gradients 3-6 % faster, weight gradients 1-7 %, forward
// products 4-11 %.
// Outputs of the fused gate|up projection + SwiGLU: h = silu(gate) * up
// ([M, F] bf16); the GEMM's own output (gate|up, [M, 2F]) goes to GemmArgs::C
// when that is not null.
struct SwigluOut {
  uint16_t* h;
  int64_t ldh;
  int64_t F;
};

// RoPE applied in the epilogue of the fused QKV projection: columns below
// nrope are heads of 128 rotated with the bf16 cos/sin tables ([>= S, 128]),
// at position m % S of output row m.
struct RopeIn {
  const uint16_t* cos;
  const uint16_t* sin;
  int64_t S;
  int64_t nrope;
};

// The fused SwiGLU backward on the down projection's input gradient: the
// GEMM's product dm = dy . W_down ([M, F]) meets gate and up in gu ([M, 2F]:
// gate columns [0, F), up columns [F, 2F)) and the epilogue writes dgate and
// dup to the same columns of dgu.
struct SwigluBwdIn {
  const uint16_t* gu;
  int64_t ldgu;
  uint16_t* dgu;
  int64_t lddgu;
  int64_t F;
};

enum { kEpiPlain = 0, kEpiSwiGLU = 1, kEpiRope = 2, kEpiSwiGLUBwd = 3, kEpiRope64 = 4 };

template <int BM, int BN, int WM, int WN>
__device__ __forceinline__ void store_swiglu(const GemmArgs& g, const SwigluOut& o,
                                             f32x4_t (&acc)[BM / WM / 16][BN / WN / 16], int64_t m0, int64_t tn,
                                             char* smem, int lane, int wave);
template <int BM, int BN, int WM, int WN, int HD>
__device__ __forceinline__ void store_rope(const GemmArgs& g, const RopeIn& r,
                                           f32x4_t (&acc)[BM / WM / 16][BN / WN / 16], int64_t m0, int64_t n0,
                                           char* smem, int lane, int wave);
template <int BM, int BN, int WM, int WN>
__device__ __forceinline__ void store_swiglu_bwd(const SwigluBwdIn& sb, f32x4_t (&acc)[BM / WM / 16][BN / WN / 16],
                                                 int64_t m0, int64_t n0, char* smem, int lane, int wave);

// One workgroup's 256 x BN tile of the direct-to-LDS GEMM (main loop, then
// the epilogue).  kEpiSwiGLU: the tile's 256 B rows are 128 gate rows and the
// matching 128 up rows of a [gate; up] weight (o.F rows apart), and the
// epilogue writes silu(gate) * up.  kEpiRope / kEpiRope64: the epilogue
// rotates the tile's columns below r.nrope as RoPE heads of 128 / 64.  kEpiSwiGLUBwd: the product is
// the down projection's input gradient and the epilogue runs SwiGLU's
// backward on it (sb).  BN = 192 (plain epilogue only): waves of 128x48.
template <typename F, int WM, int WN, bool AK, bool BK, int DBK, int NST, int kEpi, int BN = 256>
__device__ __forceinline__ void gemm_dma_tile(const GemmArgs& g, const SwigluOut& o, const RopeIn& rope,
                                              const SwigluBwdIn& sb) {
  constexpr bool kSwiGLU = kEpi == kEpiSwiGLU;
  constexpr int BM = 256, MI = 16;
  constexpr int kWaves = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / MI, FN = TN / MI;
  constexpr int kAOpBytes = BM * DBK * 2, kBOpBytes = BN * DBK * 2;  // one operand, one stage
  constexpr int kStage = kAOpBytes + kBOpBytes;
  constexpr int kLoadWaves = kWaves / 2;                // waves that issue the stage loads
  constexpr int kPerWaveA = kAOpBytes / 1024 / kLoadWaves;  // wave loads per operand per stage
  constexpr int kPerWaveB = kBOpBytes / 1024 / kLoadWaves;
  static_assert(DBK == 64 && NST == 2, "two LDS stages of 64 K: two 32-deep slices each");
  static_assert(BN == 256 || (BN == 192 && kEpi == kEpiPlain), "256-wide tiles, or 192-wide with the plain epilogue");
  static_assert(kPerWaveA * kLoadWaves * 1024 == kAOpBytes && kPerWaveB * kLoadWaves * 1024 == kBOpBytes,
                "operand stages must split evenly over the waves");
  static_assert(kWaves * MI * (TN + 4) * 4 <= NST * kStage, "epilogue staging does not fit");
  static_assert(kWaves * epi_wave_bytes<TM, TN>() <= NST * kStage, "epilogue staging does not fit");
  static_assert(kEpi == kEpiPlain || F::kDtype == LZ_BF16, "the fused epilogues are bf16");

  __shared__ __attribute__((aligned(1024))) char smem[NST * kStage];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it stay scalar
  const int wm = wave / WN, wn = wave % WN;
  const int64_t tiles_m = lz_cdiv(g.M, BM), tiles_n = lz_cdiv(g.N, BN);
  int64_t tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = tm * BM, n0 = tn * BN;
  const int64_t kbeg = (int64_t)blockIdx.y * g.kper, kend = min(g.K, kbeg + g.kper);
  const int ktiles = kend > kbeg ? (int)((kend - kbeg) / DBK) : 0;

  DmaOperand<AK, kPerWaveA, DBK> la;
  DmaOperand<BK, kPerWaveB, DBK, BN> lb;
  const int lwave = wave % kLoadWaves;     // this wave's part of a stage
  const bool loader = wave < kLoadWaves;  // wave-uniform
  la.init(g.A, g.lda, m0, g.M, kbeg, lwave, lane);
  if constexpr (kSwiGLU) lb.init(g.B, g.ldb, tn * 128, g.N, kbeg, lwave, lane, o.F);
  else lb.init(g.B, g.ldb, n0, g.N, kbeg, lwave, lane);
  DmaFrags<AK, FM> fra;
  DmaFrags<BK, FN, BN> frb;
  fra.init(wm * FM, lane);
  frb.init(wn * FN, lane);

  f32x4_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.f;

  constexpr int kReads = FN * (BK ? 1 : 2) + FM * (AK ? 1 : 2);  // LDS read instructions per slice
  if (ktiles > 0 && loader) {
    la.issue(smem, lwave, 0);
    lb.issue(smem + kAOpBytes, lwave, 0);
  }
  dma_barrier();
  if (ktiles > 1 && loader) {
    la.issue(smem + kStage, lwave, 1);
    lb.issue(smem + kStage + kAOpBytes, lwave, 1);
  }
  // slice 0 of stage kt is in registers when step kt begins
  bf16x8_t fa0[FN], fb0[FM];
  dma_load_frags(fra, frb, smem, smem + kAOpBytes, 0, fa0, fb0);
  for (int kt = 0; kt < ktiles; ++kt) {
    const char* sa = smem + (kt & 1) * kStage;
    const char* sb = sa + kAOpBytes;
    bf16x8_t fa1[FN], fb1[FM];
    dma_mfma<F>(acc, fa0, fb0);
    dma_load_frags(fra, frb, sa, sb, 1, fa1, fb1);
    sched_slice<kReads, FM * FN>();
    // this wave's loads of stage kt+1 and its reads of stage kt are done;
    // past the barrier stage kt+1 is complete and no wave reads stage kt's
    // slot any more, so stage kt+2 may refill it
    dma_barrier();
    if (kt + 2 < ktiles && loader) {
      char* nxt = smem + (kt & 1) * kStage;
      la.issue(nxt, lwave, kt + 2);
      lb.issue(nxt + kAOpBytes, lwave, kt + 2);
    }
    // slice 0 of stage kt+1 (after the last step: unused reads of the other
    // slot) while the MFMAs of slice 1 run
    const char* na = smem + ((kt + 1) & 1) * kStage;
    dma_mfma<F>(acc, fa1, fb1);
    dma_load_frags(fra, frb, na, na + kAOpBytes, 0, fa0, fb0);
    sched_slice<kReads, FM * FN>();
  }
  __syncthreads();  // every wave is done with the stages before the epilogue may reuse LDS

  if constexpr (kSwiGLU) {
    store_swiglu<BM, BN, WM, WN>(g, o, acc, m0, tn, smem, lane, wave);
  } else if constexpr (kEpi == kEpiRope || kEpi == kEpiRope64) {
    store_rope<BM, BN, WM, WN, kEpi == kEpiRope ? 128 : 64>(g, rope, acc, m0, n0, smem, lane, wave);
  } else if constexpr (kEpi == kEpiSwiGLUBwd) {
    store_swiglu_bwd<BM, BN, WM, WN>(sb, acc, m0, n0, smem, lane, wave);
  } else {
    GemmArgs go = g;  // split-K: this split's fp32 slab
    if (g.slab) go.C = static_cast<float*>(g.C) + (int64_t)blockIdx.y * g.slab;
    store_tile<F, MI, BM, BN, WM, WN>(go, acc, m0, n0, smem, lane, wave);
  }
}

template <typename F, int WM, int WN, bool AK, bool BK, int DBK, int NST>
__global__ void __launch_bounds__(64 * WM * WN) gemm_dma_kernel(GemmArgs g) {
  gemm_dma_tile<F, WM, WN, AK, BK, DBK, NST, kEpiPlain>(g, SwigluOut{}, RopeIn{}, SwigluBwdIn{});
}

// 256x192 tiles (A K-major; B either layout; plain epilogue): for products
// whose 256-wide tiles would leave CUs idle, e.g. N = 768 over 16384 rows,
// where 4 column tiles of 192 make 256 workgroups and 3 of 256 only 192.
template <typename F, bool BK>
__global__ void __launch_bounds__(512) gemm_dma_n192_kernel(GemmArgs g) {
  gemm_dma_tile<F, 2, 4, true, BK, 64, 2, kEpiPlain, 192>(g, SwigluOut{}, RopeIn{}, SwigluBwdIn{});
}

// Fused gate|up projection + SwiGLU (both operands K-major): tile (tm, tn)
// covers rows 256 tm.. of x and gate/up columns 128 tn.. of the [M, F] result.
__global__ void __launch_bounds__(512) gemm_swiglu_kernel(GemmArgs g, SwigluOut o) {
  gemm_dma_tile<FmtBF16, 2, 4, true, true, 64, 2, kEpiSwiGLU>(g, o, RopeIn{}, SwigluBwdIn{});
}

// Fused QKV projection + RoPE on the q and k heads (both operands K-major,
// M and N multiples of 256, head dim HD = 128 or 64).
template <int HD>
__global__ void __launch_bounds__(512) gemm_rope_kernel(GemmArgs g, RopeIn r) {
  gemm_dma_tile<FmtBF16, 2, 4, true, true, 64, 2, HD == 128 ? kEpiRope : kEpiRope64>(g, SwigluOut{}, r, SwigluBwdIn{});
}

// Down projection input gradient + SwiGLU backward (dy K-major, W_down read
// N-major; M and F multiples of 256).
__global__ void __launch_bounds__(512) gemm_swiglu_bwd_kernel(GemmArgs g, SwigluBwdIn sb) {
  gemm_dma_tile<FmtBF16, 2, 4, true, false, 64, 2, kEpiSwiGLUBwd>(g, SwigluOut{}, RopeIn{}, sb);
}

// SwiGLU backward epilogue.  Each wave parks its 128x64 tile of dm, rounded
// to bf16 as the GEMM's own output would be, in its LDS region (the layout
// store_tile16 uses), then walks it in 16-byte row pieces: with the gate and
// up pieces at the same row and columns it forms dgate and dup exactly as the
// unfused SwiGLU backward kernel does (the same element routine) and writes
// them as whole 16-byte pieces.
template <int BM, int BN, int WM, int WN>
__device__ __forceinline__ void store_swiglu_bwd(const SwigluBwdIn& sb, f32x4_t (&acc)[BM / WM / 16][BN / WN / 16],
                                                 int64_t m0, int64_t n0, char* smem, int lane, int wave) {
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 16, FN = TN / 16;
  constexpr int kRow = TN * 2, kChunks = kRow / 16;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t mrow0 = m0 + wm * TM, ncol0 = n0 + wn * TN;
  char* st = smem + wave * (TM * TN * 2);
  park16<FmtBF16, 16, FM, FN, kRow>(acc, st, lane, 1.0f);
  asm volatile("" ::: "memory");
  constexpr int kIters = TM * kChunks / 64;
  constexpr int kBlk = 16;  // every gate and up piece of the wave's tile loaded together (acc is free after the park)
  static_assert(kIters % kBlk == 0, "store blocks must tile the wave's rows");
#pragma unroll
  for (int t0 = 0; t0 < kIters; t0 += kBlk) {
    uint4 gv[kBlk], uv[kBlk];
#pragma unroll
    for (int u = 0; u < kBlk; ++u) {
      const int idx = (t0 + u) * 64 + lane, row = idx / kChunks, chunk = idx % kChunks;
      const uint16_t* gp = sb.gu + (mrow0 + row) * sb.ldgu + ncol0 + chunk * 8;
      gv[u] = *reinterpret_cast<const uint4*>(gp);
      uv[u] = *reinterpret_cast<const uint4*>(gp + sb.F);
    }
#pragma unroll
    for (int u = 0; u < kBlk; ++u) {
      const int idx = (t0 + u) * 64 + lane, row = idx / kChunks, chunk = idx % kChunks;
      const uint4 hv = *reinterpret_cast<const uint4*>(st + epi_off<kRow>(row, chunk));
      uint4 dg, du;
      swiglu_bwd8(gv[u], uv[u], hv, dg, du);
      uint16_t* dp = sb.dgu + (mrow0 + row) * sb.lddgu + ncol0 + chunk * 8;
      st_nt16(dp, dg);
      st_nt16(dp + sb.F, du);
    }
  }
}

// SwiGLU epilogue.  Each wave stages its 128x64 tile as bf16 in its own LDS
// region (the layout store_tile16 uses), optionally writes it to gate|up,
// then, after a workgroup barrier, the gate wave (wn = 0, 1) and the up wave
// with the same columns (wn + 2) each take half of the rows: h is computed
// from the two staged bf16 tiles exactly as the unfused SwiGLU kernel does
// from the stored gate|up, and written as whole 128-byte rows.
template <int BM, int BN, int WM, int WN>
__device__ __forceinline__ void store_swiglu(const GemmArgs& g, const SwigluOut& o,
                                             f32x4_t (&acc)[BM / WM / 16][BN / WN / 16], int64_t m0, int64_t tn,
                                             char* smem, int lane, int wave) {
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 16, FN = TN / 16;
  static_assert(WN == 4 && TN == 64, "gate and up are two 64-column waves each");
  constexpr int kRow = TN * 2, kChunks = kRow / 16, kWaveBytes = TM * kRow;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t mrow0 = m0 + wm * TM;
  const int64_t col = tn * 128 + (wn & 1) * 64;  // gate (and up) column of this wave's tile
  char* st = smem + wave * kWaveBytes;
  park16<FmtBF16, 16, FM, FN, kRow>(acc, st, lane, 1.0f);
  if (g.C) {
    asm volatile("" ::: "memory");
    uint16_t* gu = static_cast<uint16_t*>(g.C) + (wn < 2 ? 0 : o.F) + col;
#pragma unroll
    for (int t = 0; t < TM * kChunks / 64; ++t) {
      const int idx = t * 64 + lane, row = idx / kChunks, chunk = idx % kChunks;
      const uint4 v = *reinterpret_cast<const uint4*>(st + epi_off<kRow>(row, chunk));
      st_nt16(gu + (mrow0 + row) * g.ldc + chunk * 8, v);
    }
  }
  __syncthreads();
  const int gw = wn < 2 ? wave : wave - 2;  // the gate wave of this pair
  const char* sg = smem + gw * kWaveBytes;
  const char* su = sg + 2 * kWaveBytes;
  const int r0 = wn < 2 ? 0 : TM / 2;
#pragma unroll
  for (int t = 0; t < (TM / 2) * kChunks / 64; ++t) {
    const int idx = t * 64 + lane, row = r0 + idx / kChunks, chunk = idx % kChunks;
    const int off = epi_off<kRow>(row, chunk);
    const uint4 gv = *reinterpret_cast<const uint4*>(sg + off);
    const uint4 uv = *reinterpret_cast<const uint4*>(su + off);
    st_nt16(o.h + (mrow0 + row) * o.ldh + col + chunk * 8, swiglu_fwd8(gv, uv));
  }
}

// RoPE epilogue.  Tiles at or past nrope (the v heads) take the plain store.
// Otherwise each wave stages its 128x64 bf16 tile (the rounded GEMM output)
// in LDS; after a workgroup barrier the waves holding the two halves of one
// head (wn = 2j: columns 0-63 = x1, wn = 2j+1: columns 64-127 = x2) each take
// half of the rows and write
//   y1 = r(r(x1*c) + r(-x2*s)),  y2 = r(r(x2*c) + r(x1*s))
// with the table row of the output row's position: the reference's bf16
// per-op rounding, as the RoPE kernel computes it.
// RoPE on 8 (x1, x2) pairs of bf16 values with their cos/sin table pieces
// (c1, n1 at x1's columns, c2, n2 at x2's): each product rounded to bf16,
// then the sum, as the reference's separate bf16 ops round them.
__device__ __forceinline__ void rope_pair8(const uint4& av, const uint4& bv, const uint4& c1, const uint4& c2,
                                           const uint4& n1, const uint4& n2, uint4& y1, uint4& y2) {
  const uint32_t aw[4] = {av.x, av.y, av.z, av.w}, bw[4] = {bv.x, bv.y, bv.z, bv.w};
  const uint32_t c1w[4] = {c1.x, c1.y, c1.z, c1.w}, c2w[4] = {c2.x, c2.y, c2.z, c2.w};
  const uint32_t s1w[4] = {n1.x, n1.y, n1.z, n1.w}, s2w[4] = {n2.x, n2.y, n2.z, n2.w};
  uint32_t o1w[4], o2w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float o1[2], o2[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float a = bf2f((uint16_t)(aw[k] >> (16 * e))), b = bf2f((uint16_t)(bw[k] >> (16 * e)));
      const float cc1 = bf2f((uint16_t)(c1w[k] >> (16 * e))), cc2 = bf2f((uint16_t)(c2w[k] >> (16 * e)));
      const float ss1 = bf2f((uint16_t)(s1w[k] >> (16 * e))), ss2 = bf2f((uint16_t)(s2w[k] >> (16 * e)));
      o1[e] = __fadd_rn(round_bf(__fmul_rn(a, cc1)), round_bf(__fmul_rn(-b, ss1)));
      o2[e] = __fadd_rn(round_bf(__fmul_rn(b, cc2)), round_bf(__fmul_rn(a, ss2)));
    }
    o1w[k] = pack_bf16x2(o1[0], o1[1]);
    o2w[k] = pack_bf16x2(o2[0], o2[1]);
  }
  y1 = make_uint4(o1w[0], o1w[1], o1w[2], o1w[3]);
  y2 = make_uint4(o2w[0], o2w[1], o2w[2], o2w[3]);
}

template <int BM, int BN, int WM, int WN, int HD>
__device__ __forceinline__ void store_rope(const GemmArgs& g, const RopeIn& r,
                                           f32x4_t (&acc)[BM / WM / 16][BN / WN / 16], int64_t m0, int64_t n0,
                                           char* smem, int lane, int wave) {
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 16, FN = TN / 16;
  static_assert(WN == 4 && TN == 64, "a head of 128 is two 64-column waves, a head of 64 one");
  static_assert(HD == 128 || HD == 64, "heads of 128 or 64");
  if (n0 >= r.nrope) {
    store_tile<FmtBF16, 16, BM, BN, WM, WN>(g, acc, m0, n0, smem, lane, wave);
    return;
  }
  constexpr int kRow = TN * 2, kChunks = kRow / 16, kWaveBytes = TM * kRow, kHd = 2 * TN;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t mrow0 = m0 + wm * TM;
  char* st = smem + wave * kWaveBytes;
  park16<FmtBF16, 16, FM, FN, kRow>(acc, st, lane, 1.0f);
  if constexpr (HD == 64) {
    // A head is the wave's own 64 columns: x1 in chunks 0-3 and x2 in chunks
    // 4-7 of each parked row, so the wave reads back only its own region.
    asm volatile("" ::: "memory");
    constexpr int kHalf = kChunks / 2;
    uint16_t* out = static_cast<uint16_t*>(g.C) + n0 + wn * TN;
    const int64_t pos0 = mrow0 % r.S;
#pragma unroll
    for (int t = 0; t < TM * kHalf / 64; ++t) {
      const int idx = t * 64 + lane, row = idx / kHalf, chunk = idx % kHalf;
      const uint4 av = *reinterpret_cast<const uint4*>(st + epi_off<kRow>(row, chunk));
      const uint4 bv = *reinterpret_cast<const uint4*>(st + epi_off<kRow>(row, chunk + kHalf));
      int64_t pos = pos0 + row;
      while (pos >= r.S) pos -= r.S;
      const int64_t tab = pos * HD + chunk * 8;
      const uint4 c1 = *reinterpret_cast<const uint4*>(r.cos + tab), c2 = *reinterpret_cast<const uint4*>(r.cos + tab + HD / 2);
      const uint4 n1 = *reinterpret_cast<const uint4*>(r.sin + tab), n2 = *reinterpret_cast<const uint4*>(r.sin + tab + HD / 2);
      uint4 y1, y2;
      rope_pair8(av, bv, c1, c2, n1, n2, y1, y2);
      uint16_t* dst = out + (mrow0 + row) * g.ldc + chunk * 8;
      st_nt16(dst, y1);
      st_nt16(dst + HD / 2, y2);
    }
    return;
  }
  __syncthreads();
  const int xw = wave & ~1;  // the wave holding x1 of this head
  const char* s1 = smem + xw * kWaveBytes;
  const char* s2 = s1 + kWaveBytes;
  const int r0 = (wn & 1) ? TM / 2 : 0;
  uint16_t* out = static_cast<uint16_t*>(g.C) + n0 + (wn >> 1) * kHd;
  // position of the wave's first row; later rows count up from it (one
  // division per wave, not one per row)
  const int64_t pos0 = (mrow0 + r0) % r.S;
#pragma unroll
  for (int t = 0; t < (TM / 2) * kChunks / 64; ++t) {
    const int idx = t * 64 + lane, row = r0 + idx / kChunks, chunk = idx % kChunks;
    const int off = epi_off<kRow>(row, chunk);
    const uint4 av = *reinterpret_cast<const uint4*>(s1 + off);
    const uint4 bv = *reinterpret_cast<const uint4*>(s2 + off);
    const int64_t m = mrow0 + row;
    int64_t pos = pos0 + (row - r0);  // below pos0 + TM / 2
    while (pos >= r.S) pos -= r.S;    // once at most for S >= TM / 2
    const int64_t tab = pos * kHd + chunk * 8;
    const uint4 c1 = *reinterpret_cast<const uint4*>(r.cos + tab), c2 = *reinterpret_cast<const uint4*>(r.cos + tab + TN);
    const uint4 n1 = *reinterpret_cast<const uint4*>(r.sin + tab), n2 = *reinterpret_cast<const uint4*>(r.sin + tab + TN);
    uint4 y1, y2;
    rope_pair8(av, bv, c1, c2, n1, n2, y1, y2);
    uint16_t* dst = out + m * g.ldc + chunk * 8;
    st_nt16(dst, y1);
    st_nt16(dst + TN, y2);
  }
}

// Sums the fp32 partial slabs of a split-K product and applies the epilogue
// (alpha, beta*C, R) to the real output, 4 columns per thread, in a fixed
// order so results do not depend on scheduling.
template <typename F>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(GemmArgs g, const float* __restrict__ slabs, int splits) {
  const int64_t n4 = lz_cdiv(g.N, 4);
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= g.M * n4) return;
  const int64_t m = idx / n4, n = (idx - m * n4) * 4;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  const int64_t mn = g.M * g.N;
  if (g.N % 4 == 0) {  // 16-byte slab reads (the workspace is 16-byte aligned)
    for (int sp = 0; sp < splits; ++sp) {
      const float4 x = *reinterpret_cast<const float4*>(slabs + sp * mn + m * g.N + n);
      v[0] += x.x;
      v[1] += x.y;
      v[2] += x.z;
      v[3] += x.w;
    }
  } else {
    for (int sp = 0; sp < splits; ++sp) {
      const float* row = slabs + sp * mn + m * g.N;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < g.N) v[e] += row[n + e];
    }
  }
  store_out4<F>(g, m, n, v);
}

// Tile configurations: 0 = 256x256 with 8 waves (128x64 per wave),
// 1 = 256x256 with 4 waves (128x128 per wave, accumulators in AGPRs),
// 2 = 128x128 with 4 waves; 5 = the direct-to-LDS kernel (any layouts,
// 8 waves, two stages of 64 K); 6 = the direct-to-LDS kernel on 256x192
// tiles (K-major A, unsplit).
struct Plan {
  int cfg;
  int splits;
  int64_t kper;
};

// Main-loop time of a 256x192 tile relative to a 256x256 one (its MFMAs are
// three quarters, its A stage the same).
constexpr double kTile192 = 0.8;

// Rounds of `tiles` workgroups over the CUs with a partial last round counted
// by the square root of its fill: tiles of a short last round run faster than
// those of a full one.  Measured on MI355X: at 16384x1280x768, 320 tiles of
// 256x256 (1.25 rounds) beat 448 of 256x192 (1.75) by 5 %; at 16384x768xK,
// 256 tiles of 256x192 beat 192 of 256x256 by 2-8 % (K = 768 ... 4096).
inline double fill_rounds(int64_t tiles, int cus) {
  return (double)(tiles / cus) + std::sqrt((double)(tiles % cus) / (double)cus);
}

Plan make_plan(int64_t M, int64_t N, int64_t K, bool ak, bool bk) {
  const int cus = lz_num_cus();
  const int64_t big = lz_cdiv(M, 256) * lz_cdiv(N, 256);
  const int64_t small = lz_cdiv(M, 128) * lz_cdiv(N, 128);
  const int64_t mid = lz_cdiv(M, 256) * lz_cdiv(N, 192);
  // 256x256 tiles: the direct-to-LDS kernel whenever every split is a whole
  // number of 64-deep K steps; otherwise the register-staged kernel (8 waves
  // for a K-major A, 4 waves when both operands are transposed in registers).
  const int big_cfg = K % 64 == 0 ? 5 : (ak ? 0 : 1);
  Plan p{big_cfg, 1, K};
  // Cost of an unsplit product in units of one 64-deep K step of one 256x256
  // tile on one CU (about 2 us): the grid's rounds over the CUs times the
  // steps of a tile plus 2 for its prologue and epilogue.
  const double steps = (double)lz_cdiv(K, 64);
  const double c256 = (double)lz_cdiv(big, cus) * (steps + 2.0);
  double cost_cur = c256;  // of the plan so far
  if (ak && bk) {
    // 128x128 tiles (two per CU) win when they fill the chip in fewer rounds.
    // Relative speeds per tile measured on MI355X: 1.0 for the direct-to-LDS
    // 256x256 kernel and 0.75 for the 128x128 one (at the 125M QKV shape,
    // 16384x1280x768, the 256x256 kernel's two rounds beat three 128x128 ones).
    const double c128 = (double)lz_cdiv(small, 2 * cus) * (steps + 2.0) * 0.5 / 0.75 * (big_cfg == 5 ? 1.0 : 0.85);
    if (c128 < c256) {
      p.cfg = 2;
      cost_cur = c128;
    }
  }
  // The direct-to-LDS kernel adds each K step to 32-bit buffer offsets from
  // the tile's origin (a per-step base would need a scalar written by a
  // vector instruction right before the loads), so an M/N-major operand's
  // split, K rows of ld >= M (N) elements, must stay under 2^30 elements:
  // a longer K is split at least this many ways (the 7B model's weight
  // gradients over 131072 tokens: 11008 x 131072 elements, two splits).
  int min_splits = 1;
  if (big_cfg == 5) {
    const int64_t wide = std::max(ak ? (int64_t)0 : M, bk ? (int64_t)0 : N);
    if (wide > 0) {
      const int64_t kmax = (((1ll << 30) - 256) / wide) / 64 * 64;
      min_splits = kmax >= 64 ? (int)std::min<int64_t>(lz_cdiv(K, kmax), 64) : 64;
    }
  }
  if (p.cfg != 2 && K >= 1024) {
    // Long K: split it when that fills the chip better.  Same unit; a split
    // product also pays its fp32 slabs' round trip through HBM (written by
    // the product, read by the reduce: about 2 MB of slab per unit), the
    // reduce's output write (about 10 MB per unit) and 3 units for the
    // reduce launch.  Fitted to weight-gradient sweeps over K = 16384 on
    // MI355X (768x768 ... 2048x5632 outputs, 1 ... 32 splits), whose measured
    // order of plans it reproduces: e.g. 768x768 is fastest at 16 splits
    // (42 us; 26 splits 50 us), 2048x5632 unsplit (1.2 PFLOP/s; 4 splits
    // 1.05).  Splits are whole multiples of 64 in K and at least 256 deep.
    const double mn = (double)M * (double)N;
    double best = 1e30;
    for (int sp = 1; sp <= 32; ++sp) {
      const int64_t kper = lz_cdiv(lz_cdiv(K, sp), 64) * 64;
      if (sp > 1 && kper < 256) break;
      if (lz_cdiv(K, kper) != sp || sp < min_splits) continue;
      double cost = (double)lz_cdiv(big * sp, cus) * (double)(kper / 64 + 2);
      if (sp > 1) cost += sp * mn * 4.0 / 2e6 + mn * 4.0 / 10e6 + 3.0;
      if (cost < best - 1e-9) {
        best = cost;
        p.splits = sp;
        p.kper = kper;
      }
    }
    if (best < 1e30) cost_cur = best;
  }
  if (big_cfg == 5 && ak && min_splits == 1) {  // the plan so far: 256x256 or 128x128 tiles
    // Unsplit 256x192 tiles when they take fewer tile-steps than the plan so
    // far: N = 768 over 16384 rows is one full round of 256 tiles instead of
    // three quarters of one, each tile a quarter narrower.  Against an
    // unsplit 256x256 plan both count partial rounds by fill_rounds.
    const bool plain = p.cfg == 5 && p.splits == 1;
    const double c192 = (plain ? fill_rounds(mid, cus) : (double)lz_cdiv(mid, cus)) * (kTile192 * steps + 2.0);
    if (plain) cost_cur = fill_rounds(big, cus) * (steps + 2.0);
    if (c192 < 0.97 * cost_cur) {
      p.cfg = 6;
      p.splits = 1;
      p.kper = K;
    }
  }
  return p;
}

int64_t plan_workspace(const Plan& p, int64_t M, int64_t N) { return p.splits > 1 ? p.splits * M * N * 4 : 0; }

// Whether the direct-to-LDS kernel's buffer offsets (bytes from a tile's
// origin, 32-bit, kept below 2^31) cover an operand: a K-major operand spans
// `rows` rows of ld plus the split's K; an M/N-major one the split's K rows of
// ld.
inline bool dma_span_fits(bool kmajor, int64_t ld, int64_t kper, int64_t rows = 256) {
  const int64_t elems = kmajor ? rows * ld + kper : kper * ld + 256;
  return elems < (1ll << 30);
}

template <typename F, int BM, int BN, int WM, int WN, bool AK, bool BK>
int launch(const GemmArgs& g, int splits, hipStream_t s) {
  const int64_t tiles = lz_cdiv(g.M, BM) * lz_cdiv(g.N, BN);
  LZ_REQUIRE(tiles < (1ll << 31), "lz_gemm: too many tiles");
  gemm_kernel<F, BM, BN, WM, WN, AK, BK><<<dim3((unsigned)tiles, (unsigned)splits), 64 * WM * WN, 0, s>>>(g);
  return lz_check_launch("lz_gemm");
}

// Explicit instantiations: when the host pass only meets these kernels through
// the dispatch templates it does not emit the launch stubs of the variants
// that use ds_read_b64_tr_b16.
template __global__ void gemm_dma_kernel<FmtBF16, 2, 4, true, true, 64, 2>(GemmArgs);
template __global__ void gemm_dma_kernel<FmtBF16, 2, 4, true, false, 64, 2>(GemmArgs);
template __global__ void gemm_dma_kernel<FmtBF16, 2, 4, false, true, 64, 2>(GemmArgs);
template __global__ void gemm_dma_kernel<FmtBF16, 2, 4, false, false, 64, 2>(GemmArgs);
template __global__ void gemm_dma_kernel<FmtF16, 2, 4, true, true, 64, 2>(GemmArgs);
template __global__ void gemm_dma_kernel<FmtF16, 2, 4, true, false, 64, 2>(GemmArgs);
template __global__ void gemm_dma_kernel<FmtF16, 2, 4, false, true, 64, 2>(GemmArgs);
template __global__ void gemm_dma_kernel<FmtF16, 2, 4, false, false, 64, 2>(GemmArgs);
template __global__ void gemm_dma_n192_kernel<FmtBF16, true>(GemmArgs);
template __global__ void gemm_dma_n192_kernel<FmtBF16, false>(GemmArgs);
template __global__ void gemm_dma_n192_kernel<FmtF16, true>(GemmArgs);
template __global__ void gemm_dma_n192_kernel<FmtF16, false>(GemmArgs);
template __global__ void gemm_rope_kernel<128>(GemmArgs, RopeIn);
template __global__ void gemm_rope_kernel<64>(GemmArgs, RopeIn);

template <typename F, int WM, int WN, bool AK, bool BK, int DBK, int NST>
int launch_dma(const GemmArgs& g, int splits, hipStream_t s) {
  const int64_t tiles = lz_cdiv(g.M, 256) * lz_cdiv(g.N, 256);
  LZ_REQUIRE(tiles < (1ll << 31), "lz_gemm: too many tiles");
  gemm_dma_kernel<F, WM, WN, AK, BK, DBK, NST><<<dim3((unsigned)tiles, (unsigned)splits), 64 * WM * WN, 0, s>>>(g);
  return lz_check_launch("lz_gemm");
}

template <typename F, bool BK>
int launch_dma192(const GemmArgs& g, int splits, hipStream_t s) {
  const int64_t tiles = lz_cdiv(g.M, 256) * lz_cdiv(g.N, 192);
  LZ_REQUIRE(tiles < (1ll << 31), "lz_gemm: too many tiles");
  gemm_dma_n192_kernel<F, BK><<<dim3((unsigned)tiles, (unsigned)splits), 512, 0, s>>>(g);
  return lz_check_launch("lz_gemm");
}

template <typename F, bool AK, bool BK>
int dispatch(const GemmArgs& g, int cfg, int splits, hipStream_t s) {
  if (cfg == 5) return launch_dma<F, 2, 4, AK, BK, 64, 2>(g, splits, s);
  if constexpr (AK) {
    if (cfg == 6) return launch_dma192<F, BK>(g, splits, s);
  }
  switch (cfg) {
    case 0:
      return launch<F, 256, 256, 2, 4, AK, BK>(g, splits, s);
    case 1:
      return launch<F, 256, 256, 2, 2, AK, BK>(g, splits, s);
    default:
      return launch<F, 128, 128, 2, 2, AK, BK>(g, splits, s);
  }
}

template <typename F>
int dispatch_layout(const GemmArgs& g, bool ak, bool bk, int cfg, int splits, hipStream_t s) {
  if (ak && bk) return dispatch<F, true, true>(g, cfg, splits, s);
  if (ak) return dispatch<F, true, false>(g, cfg, splits, s);
  if (bk) return dispatch<F, false, true>(g, cfg, splits, s);
  return dispatch<F, false, false>(g, cfg, splits, s);
}

}  // namespace

// Workspace bytes lz_gemm uses for this shape and layout (0 when the product
// is not split along K).
LZ_EXPORT int64_t lz_gemm_workspace(int64_t M, int64_t N, int64_t K, int a_kmajor, int b_kmajor) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return plan_workspace(make_plan(M, N, K, a_kmajor != 0, b_kmajor != 0), M, N);
}

// The kernel lz_gemm launches for this shape and layout, encoded as
// 64 * cfg + splits: cfg 5 = direct-to-LDS 256x256 tile with 8 waves,
// 6 = direct-to-LDS 256x192 tile with 8 waves (unsplit),
// 0 / 1 = register-staged 256x256 with 8 / 4 waves, 2 = 128x128 with 4 waves;
// splits = number of K slices (1 = unsplit; more need the workspace).
LZ_EXPORT int lz_gemm_plan(int64_t M, int64_t N, int64_t K, int a_kmajor, int b_kmajor) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const Plan p = make_plan(M, N, K, a_kmajor != 0, b_kmajor != 0);
  return 64 * p.cfg + p.splits;
}

// C = alpha * sum_k A(m,k) B(n,k) (+ beta*C) (+ R), see the top of this file
// for the operand layouts.  A and B: ab_dtype (LZ_BF16 or LZ_F16); C: [M,N]
// in ab_dtype or fp32 (c_dtype, ldc); R: optional [M,N] in ab_dtype (ldr).  Requirements: A and B 16-byte aligned, lda and ldb multiples
// of 8; K % 8 == 0 for a K-major operand; M % 8 == 0 (N % 8 == 0) for an
// M-major A (N-major B).  `ws` (16-byte aligned, ws_bytes long, may be null)
// holds the fp32 partial products when K is split; with less workspace than
// lz_gemm_workspace() reports the product runs unsplit.
LZ_EXPORT int lz_gemm(const void* A, int64_t lda, int a_kmajor, const void* B, int64_t ldb, int b_kmajor, int ab_dtype,
                      void* C, int64_t ldc, int c_dtype, const void* R, int64_t ldr, int64_t M, int64_t N, int64_t K,
                      float alpha, float beta, void* ws, int64_t ws_bytes, void* stream) {
  LZ_REQUIRE(M >= 0 && N >= 0 && K >= 0, "lz_gemm: negative shape");
  if (M == 0 || N == 0) return LZ_OK;
  LZ_REQUIRE(A && B && C, "lz_gemm: null pointer");
  LZ_REQUIRE(lda % 8 == 0 && ldb % 8 == 0, "lz_gemm: lda (%lld) and ldb (%lld) must be multiples of 8",
             (long long)lda, (long long)ldb);
  LZ_REQUIRE((!a_kmajor && !b_kmajor) || K % 8 == 0, "lz_gemm: K (%lld) must be a multiple of 8", (long long)K);
  LZ_REQUIRE(a_kmajor || M % 8 == 0, "lz_gemm: M-major A needs M %% 8 == 0 (M = %lld)", (long long)M);
  LZ_REQUIRE(b_kmajor || N % 8 == 0, "lz_gemm: N-major B needs N %% 8 == 0 (N = %lld)", (long long)N);
  LZ_REQUIRE(lz_aligned16(A) && lz_aligned16(B), "lz_gemm: A and B must be 16-byte aligned");
  LZ_REQUIRE(lda >= (a_kmajor ? K : M) && ldb >= (b_kmajor ? K : N) && ldc >= N && (R == nullptr || ldr >= N),
             "lz_gemm: bad leading dimension");
  LZ_REQUIRE(ab_dtype == LZ_BF16 || ab_dtype == LZ_F16, "lz_gemm: bad operand dtype %d", ab_dtype);
  LZ_REQUIRE(c_dtype == ab_dtype || c_dtype == LZ_F32, "lz_gemm: bad output dtype %d for operands of dtype %d", c_dtype,
             ab_dtype);
  LZ_REQUIRE(ws_bytes >= 0 && (ws == nullptr || lz_aligned16(ws)), "lz_gemm: workspace must be 16-byte aligned");
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
  g.vec16 = ((ldc * esz) % 16 == 0) && lz_aligned16(C) &&
            (R == nullptr || ((ldr * 2) % 8 == 0 && (reinterpret_cast<uintptr_t>(R) & 7) == 0));
  g.r16 = R != nullptr && (ldr * 2) % 16 == 0 && lz_aligned16(R);
  g.vec_store = (N % 4 == 0) && (ldc % 4 == 0) && ((reinterpret_cast<uintptr_t>(C) & (4 * esz - 1)) == 0) &&
                (R == nullptr || ((ldr % 4 == 0) && (reinterpret_cast<uintptr_t>(R) & 7) == 0));
  g.kper = K > 0 ? K : 1;
  g.slab = 0;
  hipStream_t s = lz_stream(stream);
  const bool ak = a_kmajor != 0, bk = b_kmajor != 0;
  Plan p = make_plan(M, N, K, ak, bk);
  if (p.splits > 1 && (ws == nullptr || ws_bytes < plan_workspace(p, M, N))) {
    p.splits = 1;
    p.kper = g.kper;
  }
  if ((p.cfg == 5 || p.cfg == 6) && !(dma_span_fits(ak, lda, p.kper) && dma_span_fits(bk, ldb, p.kper)))
    p.cfg = ak ? 0 : 1;  // register-staged loads take 64-bit addresses
  const bool f16 = ab_dtype == LZ_F16;
  if (p.splits == 1)
    return f16 ? dispatch_layout<FmtF16>(g, ak, bk, p.cfg, 1, s) : dispatch_layout<FmtBF16>(g, ak, bk, p.cfg, 1, s);
  GemmArgs gs = g;  // partial products into fp32 slabs [splits][M][N]
  gs.C = ws;
  gs.ldc = N;
  gs.c_f32 = 1;
  gs.alpha = 1.f;
  gs.beta = 0.f;
  gs.R = nullptr;
  gs.vec_store = N % 4 == 0;
  gs.vec16 = N % 4 == 0 && lz_aligned16(ws);
  gs.kper = p.kper;
  gs.slab = M * N;
  int rc = f16 ? dispatch_layout<FmtF16>(gs, ak, bk, p.cfg, p.splits, s)
               : dispatch_layout<FmtBF16>(gs, ak, bk, p.cfg, p.splits, s);
  if (rc) return rc;
  const unsigned grid = (unsigned)lz_cdiv(M * lz_cdiv(N, 4), 256);
  if (f16) splitk_reduce_kernel<FmtF16><<<grid, 256, 0, s>>>(g, static_cast<const float*>(ws), p.splits);
  else splitk_reduce_kernel<FmtBF16><<<grid, 256, 0, s>>>(g, static_cast<const float*>(ws), p.splits);
  return lz_check_launch("lz_gemm(split-K reduce)");
}

// C = alpha * A . B^T (+ beta*C) (+ R) with A: [M,K] and B: [N,K] row-major,
// never split along K (no workspace).
LZ_EXPORT int lz_gemm_nt(const void* A, int64_t lda, const void* B, int64_t ldb, int ab_dtype, void* C, int64_t ldc,
                         int c_dtype, const void* R, int64_t ldr, int64_t M, int64_t N, int64_t K, float alpha,
                         float beta, void* stream) {
  return lz_gemm(A, lda, 1, B, ldb, 1, ab_dtype, C, ldc, c_dtype, R, ldr, M, N, K, alpha, beta, nullptr, 0, stream);
}

// Fused gate|up projection + SwiGLU (reference model/llama.py:136-146, the
// gate_proj / up_proj products and silu(gate) * up): for x [M, K] and
// w = [gate rows; up rows] ([2F, K], row-major), writes h = silu(x.Wg^T) *
// (x.Wu^T) as bf16 [M, F], and the product x.w^T itself to gu ([M, 2F]) when
// gu is not null.  Every value equals what lz_gemm (bf16 output) followed by
// lz_swiglu_fwd produces: same K order, same bf16 roundings.  Needs
// M % 256 == 0, F % 128 == 0, K % 64 == 0 and 16-byte aligned rows.
LZ_EXPORT int lz_gemm_swiglu(const void* x, int64_t ldx, const void* w, int64_t ldw, void* gu, int64_t ldgu, void* h,
                             int64_t ldh, int64_t M, int64_t F, int64_t K, void* stream) {
  LZ_REQUIRE(x && w && h, "lz_gemm_swiglu: null pointer");
  LZ_REQUIRE(M > 0 && F > 0 && K > 0 && M % 256 == 0 && F % 128 == 0 && K % 64 == 0,
             "lz_gemm_swiglu: needs M %% 256, F %% 128 and K %% 64 == 0 (M %lld, F %lld, K %lld)", (long long)M,
             (long long)F, (long long)K);
  LZ_REQUIRE(ldx >= K && ldw >= K && ldh >= F && (gu == nullptr || ldgu >= 2 * F),
             "lz_gemm_swiglu: bad leading dimension");
  LZ_REQUIRE(lz_aligned16(x) && lz_aligned16(w) && lz_aligned16(h) && (gu == nullptr || lz_aligned16(gu)) &&
                 ldx % 8 == 0 && ldw % 8 == 0 && ldh % 8 == 0 && (gu == nullptr || ldgu % 8 == 0),
             "lz_gemm_swiglu: rows must be 16-byte aligned");
  const int64_t tiles = (M / 256) * (F / 128);
  LZ_REQUIRE(tiles < (1ll << 31), "lz_gemm_swiglu: too many tiles");
  LZ_REQUIRE(dma_span_fits(true, ldx, K) && dma_span_fits(true, ldw, K, 128 + F), "lz_gemm_swiglu: operands too large");
  GemmArgs g{};
  g.A = (const uint16_t*)x;
  g.B = (const uint16_t*)w;
  g.C = gu;
  g.R = nullptr;
  g.lda = ldx;
  g.ldb = ldw;
  g.ldc = gu ? ldgu : 2 * F;
  g.ldr = 0;
  g.M = M;
  g.N = 2 * F;
  g.K = K;
  g.alpha = 1.f;
  g.beta = 0.f;
  g.c_f32 = 0;
  g.vec_store = 1;
  g.vec16 = 1;
  g.kper = K;
  g.slab = 0;
  gemm_swiglu_kernel<<<dim3((unsigned)tiles, 1), 512, 0, lz_stream(stream)>>>(g, SwigluOut{(uint16_t*)h, ldh, F});
  return lz_check_launch("lz_gemm_swiglu");
}

// Down projection input gradient fused with SwiGLU's backward (reference
// model/llama.py:136-146: autograd of down_proj(silu(gate_proj x) * up_proj
// x) in bf16): dm = dy . W_down (dy [M, K], W_down [K, F] row-major, so the
// product reads it N-major) and, with gu = [gate | up] ([M, 2F]), writes
// dgate and dup to columns [0, F) and [F, 2F) of dgu.  Every value equals
// lz_gemm (bf16 output) followed by lz_swiglu_bwd; dm itself is not stored.
// Needs M % 256 == 0, F % 256 == 0, K % 64 == 0 and 16-byte aligned rows.
LZ_EXPORT int lz_gemm_swiglu_bwd(const void* dy, int64_t lddy, const void* w, int64_t ldw, const void* gu,
                                 int64_t ldgu, void* dgu, int64_t lddgu, int64_t M, int64_t F, int64_t K,
                                 void* stream) {
  LZ_REQUIRE(dy && w && gu && dgu, "lz_gemm_swiglu_bwd: null pointer");
  LZ_REQUIRE(M > 0 && F > 0 && K > 0 && M % 256 == 0 && F % 256 == 0 && K % 64 == 0,
             "lz_gemm_swiglu_bwd: needs M %% 256, F %% 256 and K %% 64 == 0 (M %lld, F %lld, K %lld)",
             (long long)M, (long long)F, (long long)K);
  LZ_REQUIRE(lddy >= K && ldw >= F && ldgu >= 2 * F && lddgu >= 2 * F, "lz_gemm_swiglu_bwd: bad leading dimension");
  LZ_REQUIRE(lz_aligned16(dy) && lz_aligned16(w) && lz_aligned16(gu) && lz_aligned16(dgu) && lddy % 8 == 0 &&
                 ldw % 8 == 0 && ldgu % 8 == 0 && lddgu % 8 == 0,
             "lz_gemm_swiglu_bwd: rows must be 16-byte aligned");
  LZ_REQUIRE(dgu != gu, "lz_gemm_swiglu_bwd: dgu must not be gu");
  const int64_t tiles = (M / 256) * (F / 256);
  LZ_REQUIRE(tiles < (1ll << 31), "lz_gemm_swiglu_bwd: too many tiles");
  LZ_REQUIRE(dma_span_fits(true, lddy, K) && dma_span_fits(false, ldw, K), "lz_gemm_swiglu_bwd: operands too large");
  GemmArgs g{};
  g.A = (const uint16_t*)dy;
  g.B = (const uint16_t*)w;
  g.C = nullptr;
  g.R = nullptr;
  g.lda = lddy;
  g.ldb = ldw;
  g.ldc = 0;
  g.ldr = 0;
  g.M = M;
  g.N = F;
  g.K = K;
  g.alpha = 1.f;
  g.beta = 0.f;
  g.c_f32 = 0;
  g.vec_store = 1;
  g.vec16 = 1;
  g.kper = K;
  g.slab = 0;
  gemm_swiglu_bwd_kernel<<<dim3((unsigned)tiles, 1), 512, 0, lz_stream(stream)>>>(
      g, SwigluBwdIn{(const uint16_t*)gu, ldgu, (uint16_t*)dgu, lddgu, F});
  return lz_check_launch("lz_gemm_swiglu_bwd");
}

// Fused QKV projection + RoPE (reference model/llama.py:95-103: the q/k/v
// projections and apply_rotary_pos_emb on q and k): out = x.w^T ([M, N]
// bf16) with columns [0, nrope) rotated as heads of 128, row m at position
// m % S of the bf16 cos/sin tables ([>= S, 128] each, halves duplicated as
// the reference's cache is).  Every value equals lz_gemm (bf16 output)
// followed by lz_rope on those columns.  Needs M % 256 == 0, N % 256 == 0,
// nrope % 256 == 0, K % 64 == 0 and 16-byte aligned rows.
LZ_EXPORT int lz_gemm_rope_hd(const void* x, int64_t ldx, const void* w, int64_t ldw, void* out, int64_t ldo,
                              const void* cos_t, const void* sin_t, int64_t S, int64_t nrope, int64_t hd, int64_t M,
                              int64_t N, int64_t K, void* stream) {
  LZ_REQUIRE(x && w && out && cos_t && sin_t, "lz_gemm_rope: null pointer");
  LZ_REQUIRE(hd == 128 || hd == 64, "lz_gemm_rope: head dim %lld (needs 128 or 64)", (long long)hd);
  LZ_REQUIRE(M > 0 && N > 0 && K > 0 && S > 0 && M % 256 == 0 && N % 256 == 0 && K % 64 == 0,
             "lz_gemm_rope: needs M %% 256, N %% 256 and K %% 64 == 0 (M %lld, N %lld, K %lld)", (long long)M,
             (long long)N, (long long)K);
  LZ_REQUIRE(nrope >= 0 && nrope <= N && nrope % 256 == 0, "lz_gemm_rope: nrope (%lld) must be a multiple of 256 <= N",
             (long long)nrope);
  LZ_REQUIRE(ldx >= K && ldw >= K && ldo >= N, "lz_gemm_rope: bad leading dimension");
  LZ_REQUIRE(lz_aligned16(x) && lz_aligned16(w) && lz_aligned16(out) && lz_aligned16(cos_t) && lz_aligned16(sin_t) &&
                 ldx % 8 == 0 && ldw % 8 == 0 && ldo % 8 == 0,
             "lz_gemm_rope: rows must be 16-byte aligned");
  const int64_t tiles = (M / 256) * (N / 256);
  LZ_REQUIRE(tiles < (1ll << 31), "lz_gemm_rope: too many tiles");
  LZ_REQUIRE(dma_span_fits(true, ldx, K) && dma_span_fits(true, ldw, K), "lz_gemm_rope: operands too large");
  GemmArgs g{};
  g.A = (const uint16_t*)x;
  g.B = (const uint16_t*)w;
  g.C = out;
  g.R = nullptr;
  g.lda = ldx;
  g.ldb = ldw;
  g.ldc = ldo;
  g.ldr = 0;
  g.M = M;
  g.N = N;
  g.K = K;
  g.alpha = 1.f;
  g.beta = 0.f;
  g.c_f32 = 0;
  g.vec_store = 1;
  g.vec16 = 1;
  g.kper = K;
  g.slab = 0;
  const RopeIn r{(const uint16_t*)cos_t, (const uint16_t*)sin_t, S, nrope};
  if (hd == 128) gemm_rope_kernel<128><<<dim3((unsigned)tiles, 1), 512, 0, lz_stream(stream)>>>(g, r);
  else gemm_rope_kernel<64><<<dim3((unsigned)tiles, 1), 512, 0, lz_stream(stream)>>>(g, r);
  return lz_check_launch("lz_gemm_rope");
}

LZ_EXPORT int lz_gemm_rope(const void* x, int64_t ldx, const void* w, int64_t ldw, void* out, int64_t ldo,
                           const void* cos_t, const void* sin_t, int64_t S, int64_t nrope, int64_t M, int64_t N,
                           int64_t K, void* stream) {
  return lz_gemm_rope_hd(x, ldx, w, ldw, out, ldo, cos_t, sin_t, S, nrope, 128, M, N, K, stream);
}
