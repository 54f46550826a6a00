// Causal grouped-query attention, flash style, on CDNA4 matrix cores
// (reference: model/llama.py:72-133 GroupedQueryAttention.forward with
// F.scaled_dot_product_attention(is_causal=True), K/V heads shared by
// H/KV query heads through repeat_interleave).
//
// Layouts (elements):
//   q/k/v : rows b*S + s of ld elements; head h occupies [h*hd, (h+1)*hd).  The
//           three may be column ranges of one fused QKV projection.
//   o     : same row layout with H heads.
//   lse   : [B, H, S] fp32, natural-log log-sum-exp of the scaled scores.
//   *t    : transposed copies [B, heads, hd, S] (reduction index innermost).
// The kv head of query head h is h / (H/KV); K/V are never expanded.
//
// MFMA tiling (v_mfma_f32_32x32x16_bf16).  The score tile is computed as
// S^T = K . Q^T so that each lane owns one query column: row statistics need
// one cross-half shuffle, and the probabilities already sit in the B-operand
// layout for O^T += V^T . P^T (the k-slots of the two operands are the same
// permutation of the 16 keys).  The backward splits into a dK/dV pass (one
// workgroup per 128 keys of a kv head, looping over the query heads of its
// group and the query blocks at or after the diagonal) and a dQ pass (one
// workgroup per 128 queries, looping over key blocks up to the diagonal); no
// atomics, deterministic.
#include "lz_common.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t ldq, ldk, ldv;
  uint16_t* o;
  int64_t ldo;
  float* lse;
  const uint16_t* vt;  // fwd: V^T [B,KV,hd,S]
  // backward
  const uint16_t* qt;   // [B,H,hd,S]
  const uint16_t* kt;   // [B,KV,hd,S]
  const uint16_t* dout; // rows like o
  int64_t lddo;
  const uint16_t* dot;  // dO^T [B,H,hd,S]
  const float* delta;   // [B,H,S] rowsum(dO*O)
  float* delta_w;       // the same rows, written by the dQ kernel that computes them (with o as O)
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  int64_t lddq, lddk, lddv;
  // backward with RoPE folded in: bf16 tables [>= S, hd] (row = position);
  // dq and dk are then the gradients of the un-rotated q and k
  const uint16_t* rcos;
  const uint16_t* rsin;
  int B, S, H, KV;
  float scale;
};

// Workgroup -> (query block, batch, head), heaviest query blocks first.  The
// hardware deals workgroup i to XCD i % 8; when the (batch, kv head) pairs
// split evenly over the 8 XCDs, each XCD gets its own pairs, and all query
// heads of a pair's group and neighbouring query blocks run on that XCD at
// about the same time, so the K and V rows they stream are fetched into its
// L2 once instead of by workgroups spread over every XCD.
__device__ __forceinline__ void query_block_coords(int bid, int nqb, int B, int H, int KV, int& qb, int& b, int& h) {
  const int rep = H / KV, npairs = B * KV;
  if (npairs % 8 == 0) {
    const int xcd = bid % 8, j = bid / 8;
    const int per_q = (npairs / 8) * rep;  // workgroups of one query block on one XCD
    const int qr = j / per_q, rem = j - qr * per_q;
    const int pair = xcd + 8 * (rem / rep);
    b = pair / KV;
    h = (pair % KV) * rep + rem % rep;
    qb = nqb - 1 - qr;
  } else {
    const int bh = B * H;
    qb = nqb - 1 - bid / bh;
    b = (bid % bh) / H;
    h = bid % H;
  }
}

// Workgroup -> (key block, batch, kv head), first key blocks (the most
// queries at or after them) first; pairs split over XCDs as above, so the Q
// and dO rows a pair's key blocks read share an L2.
__device__ __forceinline__ void key_block_coords(int bid, int B, int KV, int& kvb, int& b, int& g) {
  const int npairs = B * KV;
  int pair;
  if (npairs % 8 == 0) {
    const int xcd = bid % 8, j = bid / 8, ppx = npairs / 8;
    kvb = j / ppx;
    pair = xcd + 8 * (j - kvb * ppx);
  } else {
    kvb = bid / npairs;
    pair = bid % npairs;
  }
  b = pair / KV;
  g = pair % KV;
}

// Elements e0..e0+7 of an accumulator -> an 8-element MFMA operand of the
// 16-bit format F (fragments travel as bf16x8_t: 16 raw bytes per lane).
template <typename F = FmtBF16>
__device__ __forceinline__ bf16x8_t pack8(const f32x16_t& v, int e0) {
  const uint4 w = make_uint4(F::pack2(v[e0], v[e0 + 1]), F::pack2(v[e0 + 2], v[e0 + 3]),
                             F::pack2(v[e0 + 4], v[e0 + 5]), F::pack2(v[e0 + 6], v[e0 + 7]));
  return __builtin_bit_cast(bf16x8_t, w);
}

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// One 32x32x16 MFMA on operands of the format F.
template <typename F>
__device__ __forceinline__ f32x16_t mfma16(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
  if constexpr (F::kDtype == LZ_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// x combined with the value of lane ^ 32 (both halves get the same result):
// v_permlane32_swap exchanges the halves of two registers without an LDS
// round trip.
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ bf16x8_t lds_frag16(const char* p) {
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(p));
}

// Two 4-element runs (8 bytes each) -> one 8-element fragment.
__device__ __forceinline__ bf16x8_t lds_frag_2x4(const char* p0, const char* p1) {
  const uint2 a = *reinterpret_cast<const uint2*>(p0);
  const uint2 b = *reinterpret_cast<const uint2*>(p1);
  return __builtin_bit_cast(bf16x8_t, make_uint4(a.x, a.y, b.x, b.y));
}

// 8 consecutive elements of a row of length `len` starting at `idx` (multiple
// of 8), zero outside [0, len).
__device__ __forceinline__ uint4 load8(const uint16_t* row, int64_t idx, int64_t len) {
  if (idx + 8 <= len && ((reinterpret_cast<uintptr_t>(row + idx) & 15) == 0))
    return *reinterpret_cast<const uint4*>(row + idx);
  uint16_t t[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) t[e] = (idx + e < len) ? row[idx + e] : (uint16_t)0;
  return make_uint4((uint32_t)t[0] | ((uint32_t)t[1] << 16), (uint32_t)t[2] | ((uint32_t)t[3] << 16),
                    (uint32_t)t[4] | ((uint32_t)t[5] << 16), (uint32_t)t[6] | ((uint32_t)t[7] << 16));
}

template <typename F = FmtBF16>
__device__ __forceinline__ void store_bf16x4(uint16_t* p, float a, float b, float c, float d) {
  uint2 w;
  w.x = (uint32_t)F::from_f(a) | ((uint32_t)F::from_f(b) << 16);
  w.y = (uint32_t)F::from_f(c) | ((uint32_t)F::from_f(d) << 16);
  *reinterpret_cast<uint2*>(p) = w;
}

// One lane's row of a dQ or dK accumulator set (columns 32*i + 8*q4 +
// 4*half + e, the MFMA output layout), times `scale`, stored as bf16 at dst.
// With RoPE tables (cs/sn: the row's position, HD values each) the stored row
// is the gradient of the un-rotated input: the gradient pair (d1, d2) of
// columns (c, c + HD/2) in the format F becomes g1 = r(r(d1*c1) + r(d2*s2)) and
// g2 = r(r(d2*c2) - r(d1*s1)), rounding each product and sum to F as the
// separate RoPE backward pass (and the reference's bf16 autograd of
// x*cos + rotate_half(x)*sin, model/llama.py:35-39) does.  Columns c and
// c + HD/2 sit in accumulator blocks i and i + HD/64 of the same lane.
template <int HD, typename F = FmtBF16>
__device__ __forceinline__ void store_grad_row(uint16_t* dst, const f32x16_t (&acc)[HD / 32], float scale, int half,
                                               const uint16_t* cs, const uint16_t* sn) {
  if (cs == nullptr) {
#pragma unroll
    for (int i = 0; i < HD / 32; ++i)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int c = i * 32 + 8 * q4 + 4 * half;
        store_bf16x4<F>(dst + c, acc[i][4 * q4] * scale, acc[i][4 * q4 + 1] * scale, acc[i][4 * q4 + 2] * scale,
                     acc[i][4 * q4 + 3] * scale);
      }
    return;
  }
  // every table value this lane needs is loaded before the first store (the
  // stores may alias the tables as far as the compiler knows, so it would
  // otherwise wait for each group's loads in turn)
  constexpr int kHalf = HD / 2, kBlk = HD / 64;
  uint2 cw[kBlk][4][2], sw[kBlk][4][2];
#pragma unroll
  for (int i = 0; i < kBlk; ++i)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int c = i * 32 + 8 * q4 + 4 * half;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        cw[i][q4][hh] = *reinterpret_cast<const uint2*>(cs + c + hh * kHalf);
        sw[i][q4][hh] = *reinterpret_cast<const uint2*>(sn + c + hh * kHalf);
      }
    }
#pragma unroll
  for (int i = 0; i < kBlk; ++i)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int c = i * 32 + 8 * q4 + 4 * half;
      const uint32_t c1a[2] = {cw[i][q4][0].x, cw[i][q4][0].y}, c2a[2] = {cw[i][q4][1].x, cw[i][q4][1].y};
      const uint32_t s1a[2] = {sw[i][q4][0].x, sw[i][q4][0].y}, s2a[2] = {sw[i][q4][1].x, sw[i][q4][1].y};
      float g1[4], g2[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int sh = (e & 1) * 16;
        const float c1 = F::to_f((uint16_t)(c1a[e >> 1] >> sh)), c2 = F::to_f((uint16_t)(c2a[e >> 1] >> sh));
        const float s1 = F::to_f((uint16_t)(s1a[e >> 1] >> sh)), s2 = F::to_f((uint16_t)(s2a[e >> 1] >> sh));
        const float d1 = F::round(acc[i][4 * q4 + e] * scale), d2 = F::round(acc[i + kBlk][4 * q4 + e] * scale);
        g1[e] = __fadd_rn(F::round(__fmul_rn(d1, c1)), F::round(__fmul_rn(d2, s2)));
        g2[e] = __fadd_rn(F::round(__fmul_rn(d2, c2)), -F::round(__fmul_rn(d1, s1)));
      }
      store_bf16x4<F>(dst + c, g1[0], g1[1], g1[2], g1[3]);
      store_bf16x4<F>(dst + c + kHalf, g2[0], g2[1], g2[2], g2[3]);
    }
}

// Row tile [rows][HD] (row stride `rb` bytes) from a [S, ld] row-major source.
template <int HD, int ROWS, int NT>
__device__ __forceinline__ void load_rows(char* dst, int rb, const uint16_t* src, int64_t ld, int64_t r0, int64_t nrows,
                                          int tid) {
  constexpr int kChunks = ROWS * HD / 8;
#pragma unroll
  for (int i = 0; i < (kChunks + NT - 1) / NT; ++i) {
    const int c = tid + i * NT;
    if (c < kChunks) {
      const int row = c / (HD / 8), ch = c % (HD / 8);
      const int64_t r = r0 + row;
      uint4 val = make_uint4(0, 0, 0, 0);
      if (r < nrows) val = *reinterpret_cast<const uint4*>(src + r * ld + ch * 8);
      *reinterpret_cast<uint4*>(dst + row * rb + ch * 16) = val;
    }
  }
}

// Transposed tile [HD][COLS] (row stride `rb` bytes, a multiple of 8) from a
// [HD, S] source, columns c0.. (zero beyond S).
template <int HD, int COLS, int NT>
__device__ __forceinline__ void load_trows(char* dst, int rb, const uint16_t* src, int64_t S, int64_t c0, int tid) {
  constexpr int kChunks = HD * COLS / 8;
#pragma unroll
  for (int i = 0; i < (kChunks + NT - 1) / NT; ++i) {
    const int c = tid + i * NT;
    if (c < kChunks) {
      const int row = c / (COLS / 8), ch = c % (COLS / 8);
      const uint4 val = load8(src + (int64_t)row * S, c0 + ch * 8, S);
      uint2* d = reinterpret_cast<uint2*>(dst + row * rb + ch * 16);
      d[0] = make_uint2(val.x, val.y);
      d[1] = make_uint2(val.z, val.w);
    }
  }
}

// ---------------------------------------------------------------------------
// Forward.  256 threads; 128 queries per workgroup (32 per wave); 64-key
// steps.  The K and V^T tiles of step i+1 are loaded into registers while step
// i computes from the other LDS buffer, so global latency overlaps the MFMAs.
// Softmax in log2 space: p = exp2(s*c - m) with c = scale*log2(e) folded into
// one FMA; O and l are rescaled only when some lane's running max moved.
// ---------------------------------------------------------------------------
template <int HD>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) attn_fwd_kernel(AttnArgs a) {
  constexpr int BQ = 128, BKV = 64, NT = 256;
  constexpr int KROW = HD * 2 + 16;
  constexpr int VROW = BKV * 2 + 8;
  constexpr int kBuf = BKV * KROW + HD * VROW;
  constexpr int kKC = BKV * HD / 8 / NT;  // 16-byte K chunks per thread per step
  constexpr int kVC = HD * BKV / 8 / NT;  // 16-byte V^T chunks per thread per step
  static_assert(kKC * NT * 8 == BKV * HD && kVC * NT * 8 == HD * BKV, "tile/thread mismatch");
  __shared__ __attribute__((aligned(16))) char smem[2 * kBuf];

  const int S = a.S, H = a.H, KV = a.KV;
  const int nqb = (S + BQ - 1) / BQ;
  int qb, b, h;
  query_block_coords(blockIdx.x, nqb, a.B, H, KV, qb, b, h);
  const int g = h / (H / KV);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, l32 = lane & 31;
  const int q0 = qb * BQ, qw0 = q0 + 32 * wave;
  const int qrow = qw0 + l32;

  bf16x8_t qf[HD / 16];
  {
    const uint16_t* qp = a.q + ((int64_t)b * S + min(qrow, S - 1)) * a.ldq + (int64_t)h * HD + 8 * half;
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) qf[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(qp + kk * 16));
  }
  f32x16_t o[HD / 32];
#pragma unroll
  for (int i = 0; i < HD / 32; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float m = -INFINITY, l = 0.f;
  const float c = a.scale * kLog2e;

  const int kv_end = min(S, q0 + BQ);
  const int kv_end_w = min(S, qw0 + 32);
  const uint16_t* kbase = a.k + (int64_t)b * S * a.ldk + (int64_t)g * HD;
  const uint16_t* vtbase = a.vt + (int64_t)(b * KV + g) * HD * S;

  uint4 kreg[kKC], vreg[kVC];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < kKC; ++i) {
      const int cidx = tid + i * NT, row = cidx / (HD / 8), ch = cidx % (HD / 8);
      const int r = k0 + row;
      const uint4 v = *reinterpret_cast<const uint4*>(kbase + (int64_t)min(r, S - 1) * a.ldk + ch * 8);
      const uint32_t msk = r < S ? ~0u : 0u;
      kreg[i] = make_uint4(v.x & msk, v.y & msk, v.z & msk, v.w & msk);
    }
#pragma unroll
    for (int i = 0; i < kVC; ++i) {
      const int cidx = tid + i * NT, row = cidx / (BKV / 8), ch = cidx % (BKV / 8);
      vreg[i] = load8(vtbase + (int64_t)row * S, k0 + ch * 8, S);
    }
  };
  auto lstore = [&](char* buf) {
#pragma unroll
    for (int i = 0; i < kKC; ++i) {
      const int cidx = tid + i * NT, row = cidx / (HD / 8), ch = cidx % (HD / 8);
      *reinterpret_cast<uint4*>(buf + row * KROW + ch * 16) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < kVC; ++i) {
      const int cidx = tid + i * NT, row = cidx / (BKV / 8), ch = cidx % (BKV / 8);
      uint2* d = reinterpret_cast<uint2*>(buf + BKV * KROW + row * VROW + ch * 16);
      d[0] = make_uint2(vreg[i].x, vreg[i].y);
      d[1] = make_uint2(vreg[i].z, vreg[i].w);
    }
  };

  const int nsteps = (kv_end + BKV - 1) / BKV;
  gload(0);
  lstore(smem);
  __syncthreads();
  for (int it = 0; it < nsteps; ++it) {
    const int k0 = it * BKV;
    if (it + 1 < nsteps) gload(k0 + BKV);
    const char* Ks = smem + (it & 1) * kBuf;
    const char* Vts = Ks + BKV * KROW;
    if (k0 < kv_end_w) {
      f32x16_t s[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[t][r] = 0.f;
#pragma unroll
        for (int kk = 0; kk < HD / 16; ++kk) {
          const bf16x8_t af = lds_frag16(Ks + (t * 32 + l32) * KROW + kk * 32 + half * 16);
          s[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, qf[kk], s[t], 0, 0, 0);
        }
      }
      const bool need_mask = (k0 + BKV - 1 > qw0) || (k0 + BKV > S);
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          if (need_mask) {
            const int kv = k0 + t * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
            if (kv > qrow || kv >= S) s[t][r] = -INFINITY;
          }
          mx = fmaxf(mx, s[t][r]);
        }
      mx = max_halves(mx);
      const float m_new = fmaxf(m, mx * c);
      const float nm = -m_new;
      float rs = 0.f;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(fmaf(s[t][r], c, nm));
          s[t][r] = p;
          rs += p;
        }
      rs = sum_halves(rs);
      if (__builtin_amdgcn_read_exec() & __ballot(m_new != m)) {  // some lane's max moved
        const float alpha = __builtin_amdgcn_exp2f(m - m_new);
        l *= alpha;
#pragma unroll
        for (int i = 0; i < HD / 32; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
      }
      l += rs;
      m = m_new;
#pragma unroll
      for (int ks = 0; ks < BKV / 16; ++ks) {
        const bf16x8_t pb = pack8(s[ks >> 1], 8 * (ks & 1));
#pragma unroll
        for (int i = 0; i < HD / 32; ++i) {
          const char* row = Vts + (i * 32 + l32) * VROW;
          const bf16x8_t av = lds_frag_2x4(row + (16 * ks + 4 * half) * 2, row + (16 * ks + 8 + 4 * half) * 2);
          o[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, pb, o[i], 0, 0, 0);
        }
      }
    }
    if (it + 1 < nsteps) lstore(smem + ((it + 1) & 1) * kBuf);
    __syncthreads();
  }
  if (qrow < S) {
    const float inv_l = 1.0f / l;
    uint16_t* op = a.o + ((int64_t)b * S + qrow) * a.ldo + (int64_t)h * HD;
#pragma unroll
    for (int i = 0; i < HD / 32; ++i)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int hd = i * 32 + 8 * q4 + 4 * half;
        store_bf16x4(op + hd, o[i][4 * q4] * inv_l, o[i][4 * q4 + 1] * inv_l, o[i][4 * q4 + 2] * inv_l,
                     o[i][4 * q4 + 3] * inv_l);
      }
    if (half == 0) a.lse[((int64_t)b * H + h) * S + qrow] = (m + log2f(l)) * kLn2;
  }
}

// ---------------------------------------------------------------------------
// Backward, dK/dV pass.  256 threads; 128 keys per workgroup (32 per wave);
// 64-query steps over every query head of the kv head's group.
// ---------------------------------------------------------------------------
template <int HD>
__global__ void __launch_bounds__(256) attn_bwd_dkdv_kernel(AttnArgs a) {
  constexpr int BKV = 128, BQ = 64, NT = 256;
  constexpr int KROW = HD * 2 + 16;
  constexpr int TROW = BQ * 2 + 8;
  __shared__ __attribute__((aligned(16))) char smem[2 * BQ * KROW + 2 * HD * TROW + 2 * BQ * 4];
  char* Qs = smem;
  char* dOs = Qs + BQ * KROW;
  char* Qts = dOs + BQ * KROW;
  char* dOts = Qts + HD * TROW;
  float* lse2s = reinterpret_cast<float*>(dOts + HD * TROW);
  float* Ds = lse2s + BQ;

  const int S = a.S, H = a.H, KV = a.KV, rep = H / KV;
  int kvb, b, g;
  key_block_coords(blockIdx.x, a.B, KV, kvb, b, g);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, l32 = lane & 31;
  const int k0 = kvb * BKV, kw0 = k0 + 32 * wave;
  const int kvrow = kw0 + l32;
  const float c = a.scale * kLog2e;

  bf16x8_t kf[HD / 16], vf[HD / 16];
  {
    const int64_t r = (int64_t)b * S + min(kvrow, S - 1);
    const uint16_t* kp = a.k + r * a.ldk + (int64_t)g * HD + 8 * half;
    const uint16_t* vp = a.v + r * a.ldv + (int64_t)g * HD + 8 * half;
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) {
      kf[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(kp + kk * 16));
      vf[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(vp + kk * 16));
    }
  }
  f32x16_t dk[HD / 32], dv[HD / 32];
#pragma unroll
  for (int i = 0; i < HD / 32; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dk[i][r] = 0.f;
      dv[i][r] = 0.f;
    }

  const int qstart = (k0 / BQ) * BQ;
  for (int hq = 0; hq < rep; ++hq) {
    const int h = g * rep + hq;
    const uint16_t* qbase = a.q + (int64_t)b * S * a.ldq + (int64_t)h * HD;
    const uint16_t* dobase = a.dout + (int64_t)b * S * a.lddo + (int64_t)h * HD;
    const uint16_t* qtbase = a.qt + (int64_t)(b * H + h) * HD * S;
    const uint16_t* dotbase = a.dot + (int64_t)(b * H + h) * HD * S;
    const float* lsep = a.lse + (int64_t)(b * H + h) * S;
    const float* dp_ = a.delta + (int64_t)(b * H + h) * S;
    for (int q0 = qstart; q0 < S; q0 += BQ) {
      load_rows<HD, BQ, NT>(Qs, KROW, qbase, a.ldq, q0, S, tid);
      load_rows<HD, BQ, NT>(dOs, KROW, dobase, a.lddo, q0, S, tid);
      load_trows<HD, BQ, NT>(Qts, TROW, qtbase, S, q0, tid);
      load_trows<HD, BQ, NT>(dOts, TROW, dotbase, S, q0, tid);
      if (tid < BQ) {
        const int q = q0 + tid;
        lse2s[tid] = q < S ? lsep[q] * kLog2e : 0.f;
        Ds[tid] = q < S ? dp_[q] : 0.f;
      }
      __syncthreads();
      if (q0 + BQ - 1 >= kw0 && kw0 < S) {
        f32x16_t s[2], dp[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            s[t][r] = 0.f;
            dp[t][r] = 0.f;
          }
#pragma unroll
          for (int kk = 0; kk < HD / 16; ++kk) {
            const bf16x8_t aq = lds_frag16(Qs + (t * 32 + l32) * KROW + kk * 32 + half * 16);
            s[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aq, kf[kk], s[t], 0, 0, 0);
            const bf16x8_t ado = lds_frag16(dOs + (t * 32 + l32) * KROW + kk * 32 + half * 16);
            dp[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ado, vf[kk], dp[t], 0, 0, 0);
          }
        }
        // lane holds key column kvrow; query rows ql = t*32 + 8*(r/4) + 4*half + r%4
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const int qlb = t * 32 + 8 * r4 + 4 * half;
            const float4 l4 = *reinterpret_cast<const float4*>(lse2s + qlb);
            const float4 d4 = *reinterpret_cast<const float4*>(Ds + qlb);
            const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
            const float dvv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int r = 4 * r4 + e;
              const int q = q0 + qlb + e;
              const bool ok = q < S && kvrow <= q && kvrow < S;
              const float p = ok ? __builtin_amdgcn_exp2f(fmaf(s[t][r], c, -lv[e])) : 0.f;
              dp[t][r] = p * (dp[t][r] - dvv[e]);
              s[t][r] = p;
            }
          }
#pragma unroll
        for (int ks = 0; ks < BQ / 16; ++ks) {
          const bf16x8_t pb = pack8(s[ks >> 1], 8 * (ks & 1));
          const bf16x8_t dsb = pack8(dp[ks >> 1], 8 * (ks & 1));
#pragma unroll
          for (int i = 0; i < HD / 32; ++i) {
            const char* dorow = dOts + (i * 32 + l32) * TROW;
            const bf16x8_t ado = lds_frag_2x4(dorow + (16 * ks + 4 * half) * 2, dorow + (16 * ks + 8 + 4 * half) * 2);
            dv[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ado, pb, dv[i], 0, 0, 0);
            const char* qrow_ = Qts + (i * 32 + l32) * TROW;
            const bf16x8_t aq = lds_frag_2x4(qrow_ + (16 * ks + 4 * half) * 2, qrow_ + (16 * ks + 8 + 4 * half) * 2);
            dk[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aq, dsb, dk[i], 0, 0, 0);
          }
        }
      }
      __syncthreads();
    }
  }
  if (kvrow < S) {
    uint16_t* dkp = a.dk + ((int64_t)b * S + kvrow) * a.lddk + (int64_t)g * HD;
    uint16_t* dvp = a.dv + ((int64_t)b * S + kvrow) * a.lddv + (int64_t)g * HD;
    const bool rope = a.rcos != nullptr;
    store_grad_row<HD>(dkp, dk, a.scale, half, rope ? a.rcos + (int64_t)kvrow * HD : nullptr,
                       rope ? a.rsin + (int64_t)kvrow * HD : nullptr);
    store_grad_row<HD>(dvp, dv, 1.0f, half, nullptr, nullptr);
  }
}

// ---------------------------------------------------------------------------
// Backward, dQ pass.  256 threads; 128 queries per workgroup; 64-key steps.
// ---------------------------------------------------------------------------
template <int HD>
__global__ void __launch_bounds__(256) attn_bwd_dq_kernel(AttnArgs a) {
  constexpr int BQ = 128, BKV = 64, NT = 256;
  constexpr int KROW = HD * 2 + 16;
  constexpr int TROW = BKV * 2 + 8;
  __shared__ __attribute__((aligned(16))) char smem[2 * BKV * KROW + HD * TROW];
  char* Ks = smem;
  char* Vs = Ks + BKV * KROW;
  char* Kts = Vs + BKV * KROW;

  const int S = a.S, H = a.H, KV = a.KV;
  const int nqb = (S + BQ - 1) / BQ;
  int qb, b, h;
  query_block_coords(blockIdx.x, nqb, a.B, H, KV, qb, b, h);
  const int g = h / (H / KV);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, l32 = lane & 31;
  const int q0 = qb * BQ, qw0 = q0 + 32 * wave;
  const int qrow = qw0 + l32;
  const int qc = min(qrow, S - 1);
  const float c = a.scale * kLog2e;

  bf16x8_t qf[HD / 16], df[HD / 16];
  {
    const uint16_t* qp = a.q + ((int64_t)b * S + qc) * a.ldq + (int64_t)h * HD + 8 * half;
    const uint16_t* dp_ = a.dout + ((int64_t)b * S + qc) * a.lddo + (int64_t)h * HD + 8 * half;
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) {
      qf[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(qp + kk * 16));
      df[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(dp_ + kk * 16));
    }
  }
  const float lse2 = a.lse[((int64_t)b * H + h) * S + qc] * kLog2e;
  const float Dq = a.delta[((int64_t)b * H + h) * S + qc];
  f32x16_t dq[HD / 32];
#pragma unroll
  for (int i = 0; i < HD / 32; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[i][r] = 0.f;

  const int kv_end = min(S, q0 + BQ);
  const int kv_end_w = min(S, qw0 + 32);
  const uint16_t* kbase = a.k + (int64_t)b * S * a.ldk + (int64_t)g * HD;
  const uint16_t* vbase = a.v + (int64_t)b * S * a.ldv + (int64_t)g * HD;
  const uint16_t* ktbase = a.kt + (int64_t)(b * KV + g) * HD * S;

  for (int k0 = 0; k0 < kv_end; k0 += BKV) {
    load_rows<HD, BKV, NT>(Ks, KROW, kbase, a.ldk, k0, S, tid);
    load_rows<HD, BKV, NT>(Vs, KROW, vbase, a.ldv, k0, S, tid);
    load_trows<HD, BKV, NT>(Kts, TROW, ktbase, S, k0, tid);
    __syncthreads();
    if (k0 < kv_end_w) {
      f32x16_t st[2], dpt[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          st[t][r] = 0.f;
          dpt[t][r] = 0.f;
        }
#pragma unroll
        for (int kk = 0; kk < HD / 16; ++kk) {
          const bf16x8_t ak = lds_frag16(Ks + (t * 32 + l32) * KROW + kk * 32 + half * 16);
          st[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ak, qf[kk], st[t], 0, 0, 0);
          const bf16x8_t av = lds_frag16(Vs + (t * 32 + l32) * KROW + kk * 32 + half * 16);
          dpt[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, df[kk], dpt[t], 0, 0, 0);
        }
      }
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kv = k0 + t * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
          const bool ok = kv <= qrow && kv < S && qrow < S;
          const float p = ok ? __builtin_amdgcn_exp2f(fmaf(st[t][r], c, -lse2)) : 0.f;
          dpt[t][r] = p * (dpt[t][r] - Dq);
        }
#pragma unroll
      for (int ks = 0; ks < BKV / 16; ++ks) {
        const bf16x8_t dsb = pack8(dpt[ks >> 1], 8 * (ks & 1));
#pragma unroll
        for (int i = 0; i < HD / 32; ++i) {
          const char* row = Kts + (i * 32 + l32) * TROW;
          const bf16x8_t ak = lds_frag_2x4(row + (16 * ks + 4 * half) * 2, row + (16 * ks + 8 + 4 * half) * 2);
          dq[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ak, dsb, dq[i], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  }
  if (qrow < S) {
    uint16_t* dqp = a.dq + ((int64_t)b * S + qrow) * a.lddq + (int64_t)h * HD;
    const bool rope = a.rcos != nullptr;
    store_grad_row<HD>(dqp, dq, a.scale, half, rope ? a.rcos + (int64_t)qrow * HD : nullptr,
                       rope ? a.rsin + (int64_t)qrow * HD : nullptr);
  }
}

// ---------------------------------------------------------------------------
// Tile path (S a multiple of 64).  Every operand tile is a [64][HD] bf16 block
// of a row-major source (Q, dO, K or V rows), copied into LDS by
// buffer_load_dwordx4 ... lds with no staging registers, in unpadded rows whose
// 16-byte chunks are XOR-swizzled by tswz().  Operands that the MFMAs need
// with the other dimension innermost (V^T, K^T, Q^T, dO^T) are read from the
// same tiles with ds_read_b64_tr_b16: within each 16-lane group, lane 4j+q
// points at row k0+j, columns n0+4q..n0+4q+3, and lane i receives column
// n0+i, rows k0..k0+3.  So no transposed copy of any operand exists in HBM.
// Two LDS stages: the tiles of step i+1 are issued right after the barrier
// that opens step i (the barrier's fence waits for the loads of step i).
// ---------------------------------------------------------------------------
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t* lds_v4i16_ptr;

// Chunk swizzle of a tile row r: keeps the 16-byte reads of 16 consecutive
// rows (row fragments) and the 8-byte transposed reads of 4 consecutive rows
// x 64 bytes (one half-wave of ds_read_b64_tr_b16) on distinct banks of the
// 64-bank LDS.
template <int HD>
__device__ __forceinline__ int tswz(int r) {
  if constexpr (HD == 128) return ((r & 3) << 2) | ((r >> 2) & 3);
  else return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
}

template <int HD>
__device__ __forceinline__ int toff(int r, int chunk) {
  return r * (HD * 2) + ((chunk ^ tswz<HD>(r)) << 4);
}

// Raw buffer starting at a tile's first row (src is the same for every
// lane): the DMA loads below take a 32-bit per-lane offset within the tile's
// 64 rows, which measured faster than 64-bit per-lane addresses.
__device__ __forceinline__ lz_v4i tile_rsrc(const uint16_t* src) { return lz_buffer_rsrc(src); }

__device__ __forceinline__ void lds_dma16(lz_v4i rsrc, uint32_t voff, char* dst) { lz_dma16(rsrc, voff, 0, dst); }

// A [64][HD] tile of rows `src` (stride ld elements) into LDS at `dst` by DMA:
// 64*HD*2/1024 wave loads split over the 4 waves.
template <int HD>
__device__ __forceinline__ void dma_tile(const uint16_t* src, int64_t ld, char* dst, int wave, int lane) {
  constexpr int kRowsPerLoad = 1024 / (HD * 2), kChunks = HD / 8;
  constexpr int kPer = 64 / kRowsPerLoad / 4;
  const lz_v4i rsrc = tile_rsrc(src);
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int r = (wave * kPer + q) * kRowsPerLoad + lane / kChunks;
    const int c = (lane % kChunks) ^ tswz<HD>(r);
    const uint32_t voff = (uint32_t)((r * ld + c * 8) * 2);
    if (q == 0) lz_dma16_first(rsrc, voff, 0, dst + (wave * kPer + q) * 1024);
    else lds_dma16(rsrc, voff, dst + (wave * kPer + q) * 1024);
  }
}

// 64 floats at src into LDS at dst by lanes 0-15 of the calling wave, and 64
// floats at src2 into dst + 256 by lanes 16-31 (src, src2 and dst uniform).
__device__ __forceinline__ void dma_rows64(const float* src, const float* src2, char* dst, int lane) {
  if (lane < 16) lz_dma16(lz_buffer_rsrc(src), 16 * lane, 0, dst);
  else if (lane < 32) lz_dma16(lz_buffer_rsrc(src2), 16 * (lane - 16), 0, dst);
}

// Per-lane LDS offsets of the fragment reads of a tile.  tswz() depends only
// on the row modulo 16, so every offset splits into a per-lane part and a
// part that only depends on the 16-row block and the 32-column block.
template <int HD>
struct TileOffsets {
  static constexpr int RB = HD * 2;
  int row;              // row fragments: (lane % 32) * RB
  int chunk[HD / 16];   // row fragments: ((2*kk + lane/32) ^ tswz) * 16
  int tbase[2];         // transposed reads 1 and 2 (rows +0 and +8)
  int tcol[HD / 32];    // transposed reads: 32-column block i

  __device__ __forceinline__ void init(int lane) {
    const int l32 = lane & 31, half = lane >> 5;
    row = l32 * RB;
    const int sw = tswz<HD>(l32);
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) chunk[kk] = ((2 * kk + half) ^ sw) << 4;
    // lane 4j+q of each 16-lane group points at row r0 + j (+8), columns
    // c0 + 16*(group % 2) + 4q .. +3
    const int p = lane & 15;
    const int col = ((lane >> 4) & 1) * 16 + 4 * (p & 3);
    const int cl = col >> 3;
    int swh = 0;
#pragma unroll
    for (int rd = 0; rd < 2; ++rd) {
      const int r = 4 * half + (p >> 2) + 8 * rd;  // row within a 16-row block
      const int swr = tswz<HD>(r);
      tbase[rd] = r * RB + ((cl ^ (swr & 3)) << 4) + (col & 7) * 2;
      swh = swr >> 2;  // the same for both reads
    }
#pragma unroll
    for (int i = 0; i < HD / 32; ++i) tcol[i] = (i ^ swh) << 6;
  }

  // Row fragment: row 32*t + lane%32, columns 16*kk + 8*(lane/32) .. +7.
  __device__ __forceinline__ bf16x8_t frag(const char* tile, int t, int kk) const {
    return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(tile + t * 32 * RB + row + chunk[kk]));
  }

  // Transposed fragment for an MFMA operand whose k index runs over tile rows:
  // lane l gets column 32*i + l%32 at rows 16*ks + 8*(e/4) + 4*(l/32) + e%4
  // for k-slots e = 0..7 (the slot order of the accumulator layout).
  __device__ __forceinline__ bf16x8_t frag_t(const char* tile, int ks, int i) const {
    const char* blk = tile + ks * 16 * RB + tcol[i];
    const v4i16_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(blk + tbase[0]));
    const v4i16_t y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(blk + tbase[1]));
    const uint2 xw = __builtin_bit_cast(uint2, x), yw = __builtin_bit_cast(uint2, y);
    return __builtin_bit_cast(bf16x8_t, make_uint4(xw.x, xw.y, yw.x, yw.y));
  }
};

// Forward on tiles: 128 queries per workgroup (32 per wave), 64-key steps,
// K and V tiles double-buffered in LDS (the next step's tiles are issued
// right after the barrier that opens a step).
template <int HD, typename F>
__device__ __forceinline__ void fwd_scores(f32x16_t (&s)[2], const TileOffsets<HD>& to, const char* Kt,
                                           const bf16x8_t (&qf)[HD / 16]) {
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[t][r] = 0.f;
#pragma unroll
  for (int kk = 0; kk < HD / 16; ++kk)
#pragma unroll
    for (int t = 0; t < 2; ++t)
      s[t] = mfma16<F>(to.frag(Kt, t, kk), qf[kk], s[t]);
}

// Online softmax of one 64-key step and its P.V product.  s: the step's
// scores (lane = query column, registers = keys t*32 + 8*(r/4) + 4*half +
// r%4); MASK: keys with index > lim are masked (the diagonal step only, so
// that the other steps carry no masking instructions).  The running max m is
// kept in log2 units; l and O are rescaled only when some lane's max moves.
template <int HD, bool MASK, typename F>
__device__ __forceinline__ void fwd_softmax_pv(f32x16_t (&s)[2], f32x16_t (&o)[HD / 32], float& m, float& l,
                                               const TileOffsets<HD>& to, const char* Vt, float c, int lim, int half) {
  constexpr int BKV = 64;
  // the V^T fragments of the first 16 keys, read now so that the first P.V
  // MFMAs do not wait for LDS after the softmax
  bf16x8_t vf[2][HD / 32];
#pragma unroll
  for (int i = 0; i < HD / 32; ++i) vf[0][i] = to.frag_t(Vt, 0, i);
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if constexpr (MASK) {
        const int kv = t * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (kv > lim) s[t][r] = -INFINITY;
      }
      mx = fmaxf(mx, s[t][r]);
    }
  mx = max_halves(mx);
  const float m_step = mx * c;
  if (__builtin_amdgcn_read_exec() & __ballot(m_step > m)) {  // some lane's max moved
    const float m_new = fmaxf(m, m_step);
    const float alpha = __builtin_amdgcn_exp2f(m - m_new);
    l *= alpha;
#pragma unroll
    for (int i = 0; i < HD / 32; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
    m = m_new;
  }
  const float nm = -m;
  float rs = 0.f;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = __builtin_amdgcn_exp2f(fmaf(s[t][r], c, nm));
      s[t][r] = p;
      rs += p;
    }
  l += sum_halves(rs);
#pragma unroll
  for (int ks = 0; ks < BKV / 16; ++ks) {
    if (ks + 1 < BKV / 16)  // the next 16 keys' fragments while these MFMAs run
#pragma unroll
      for (int i = 0; i < HD / 32; ++i) vf[(ks + 1) & 1][i] = to.frag_t(Vt, ks + 1, i);
    const bf16x8_t pb = pack8<F>(s[ks >> 1], 8 * (ks & 1));
#pragma unroll
    for (int i = 0; i < HD / 32; ++i)
      o[i] = mfma16<F>(vf[ks & 1][i], pb, o[i]);
  }
}

template <int HD, typename F>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(HD == 64 ? 4 : 2, HD == 64 ? 4 : 2))) attn_fwd_tile_kernel(AttnArgs a) {
  constexpr int BQ = 128, BKV = 64;
  constexpr int kTile = BKV * HD * 2;
  __shared__ __attribute__((aligned(1024))) char smem[4 * kTile];  // K slots 0, 1; V slots 0, 1
  char* const Ks = smem;
  char* const Vs = smem + 2 * kTile;

  const int S = a.S, H = a.H, KV = a.KV;
  const int nqb = (S + BQ - 1) / BQ;
  int qb, b, h;
  query_block_coords(blockIdx.x, nqb, a.B, H, KV, qb, b, h);
  const int g = h / (H / KV);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, l32 = lane & 31;
  TileOffsets<HD> to;
  to.init(lane);
  const int q0 = qb * BQ, qw0 = q0 + 32 * wave;
  const int qrow = qw0 + l32;

  bf16x8_t qf[HD / 16];
  {
    const uint16_t* qp = a.q + ((int64_t)b * S + min(qrow, S - 1)) * a.ldq + (int64_t)h * HD + 8 * half;
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) qf[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(qp + kk * 16));
  }
  f32x16_t o[HD / 32];
#pragma unroll
  for (int i = 0; i < HD / 32; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float m = -INFINITY, l = 0.f;
  const float c = a.scale * kLog2e;

  const int kv_end = min(S, q0 + BQ);  // a multiple of 64
  const int kv_end_w = qw0 < S ? min(S, qw0 + 32) : 0;  // a wave past the sequence computes nothing
  const uint16_t* kbase = a.k + (int64_t)b * S * a.ldk + (int64_t)g * HD;
  const uint16_t* vbase = a.v + (int64_t)b * S * a.ldv + (int64_t)g * HD;
  const int nsteps = kv_end / BKV;

  // Step it: wait for its K/V (and every wave's reads of step it-1), then
  // issue step it+1's tiles into the other slot.
  auto open_step = [&](int it) {
    dma_barrier();
    if (it + 1 < nsteps) {
      dma_tile<HD>(kbase + (int64_t)(it + 1) * BKV * a.ldk, a.ldk, Ks + ((it + 1) & 1) * kTile, wave, lane);
      dma_tile<HD>(vbase + (int64_t)(it + 1) * BKV * a.ldv, a.ldv, Vs + ((it + 1) & 1) * kTile, wave, lane);
    }
  };
  // This wave's last step holds its diagonal (the only step with masked
  // keys: 32 queries starting at a multiple of 32 against 64-key steps);
  // the loop before it has no branch, so the accumulators stay in place.
  const int last_w = kv_end_w > 0 ? (kv_end_w - 1) / BKV : -1;
  dma_tile<HD>(kbase, a.ldk, Ks, wave, lane);
  dma_tile<HD>(vbase, a.ldv, Vs, wave, lane);
  int it = 0;
  for (; it < last_w; ++it) {
    open_step(it);
    f32x16_t s[2];
    fwd_scores<HD, F>(s, to, Ks + (it & 1) * kTile, qf);
    fwd_softmax_pv<HD, false, F>(s, o, m, l, to, Vs + (it & 1) * kTile, c, 0, half);
  }
  if (last_w >= 0) {
    open_step(it);
    f32x16_t s[2];
    fwd_scores<HD, F>(s, to, Ks + (it & 1) * kTile, qf);
    fwd_softmax_pv<HD, true, F>(s, o, m, l, to, Vs + (it & 1) * kTile, c, qrow - it * BKV, half);
    ++it;
  }
  for (; it < nsteps; ++it) open_step(it);  // past this wave's diagonal: it only joins the barriers
  if (qrow < S) {
    const float inv_l = 1.0f / l;
    uint16_t* op = a.o + ((int64_t)b * S + qrow) * a.ldo + (int64_t)h * HD;
#pragma unroll
    for (int i = 0; i < HD / 32; ++i)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int hd = i * 32 + 8 * q4 + 4 * half;
        store_bf16x4<F>(op + hd, o[i][4 * q4] * inv_l, o[i][4 * q4 + 1] * inv_l, o[i][4 * q4 + 2] * inv_l,
                     o[i][4 * q4 + 3] * inv_l);
      }
    if (half == 0) a.lse[((int64_t)b * H + h) * S + qrow] = (m + log2f(l)) * kLn2;
  }
}

// A [64][HD] tile like dma_tile, loaded by the four waves of group `wg4`
// (wave index 0..3 within the group), rows past `nvalid` clamped to the last
// valid row (their results are masked).
template <int HD>
__device__ __forceinline__ void dma_tile_rows(const uint16_t* src, int64_t ld, int nvalid, char* dst, int wg4,
                                              int lane) {
  constexpr int kRowsPerLoad = 1024 / (HD * 2), kChunks = HD / 8;
  constexpr int kPer = 64 / kRowsPerLoad / 4;
  const lz_v4i rsrc = tile_rsrc(src);
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int r = (wg4 * kPer + q) * kRowsPerLoad + lane / kChunks;
    const int c = (lane % kChunks) ^ tswz<HD>(r);
    lds_dma16(rsrc, (uint32_t)((min(r, nvalid - 1) * ld + c * 8) * 2), dst + (wg4 * kPer + q) * 1024);
  }
}

// Issues the tiles of dK/dV step `step` for the 8-wave kernel: Q by waves
// 0-3, dO by waves 4-7, lse and delta by wave 0.
template <int HD>
__device__ __forceinline__ void dkdv8_issue(const AttnArgs& a, int step, int nqs, int qstart, int b, int g, int rep,
                                            char* st, int wave, int lane) {
  constexpr int kTile = 64 * HD * 2;
  const int S = a.S;
  const int hq = step / nqs, q0 = qstart + (step - hq * nqs) * 64;
  const int h = g * rep + hq;
  if (wave < 4)
    dma_tile<HD>(a.q + ((int64_t)b * S + q0) * a.ldq + (int64_t)h * HD, a.ldq, st, wave, lane);
  else
    dma_tile<HD>(a.dout + ((int64_t)b * S + q0) * a.lddo + (int64_t)h * HD, a.lddo, st + kTile, wave - 4, lane);
  if (wave == 0) {
    const int64_t off = ((int64_t)b * a.H + h) * S + q0;
    dma_rows64(a.lse + off, a.delta + off, st + 2 * kTile, lane);
  }
}

// dK/dV with two waves per SIMD: 256 keys per workgroup of 8 waves (32 keys
// per wave), K fragments in registers, the workgroup's V tile in LDS (read
// back as fragments), 64-query steps over every query head of the kv head's
// group from the diagonal on: S^T = K Q^T and dP^T = V dO^T per 32-query
// half, P = exp(S*scale - lse), dS = P (dP - delta), then dV += P^T dO and
// dK += dS^T Q from transposed LDS reads.
// One 64-query step of the 8-wave dK/dV kernel for this wave's 32 keys:
// S^T and dP^T, P and dS, then dV += P^T dO and dK += dS^T Q.  MASK: the
// step crosses this wave's diagonal, so pairs with key > query are dropped
// (the other steps carry no masking instructions).
template <int HD, bool MASK, typename F>
__device__ __forceinline__ void dkdv_step(f32x16_t (&dk)[HD / 32], f32x16_t (&dv)[HD / 32], const TileOffsets<HD>& to,
                                          const char* Qt, const char* Vt, const bf16x8_t (&kf)[HD / 16], float c,
                                          int q0, int kvrow, int wave, int half) {
  constexpr int kTile = 64 * HD * 2;
  const char* dOt = Qt + kTile;
  const float* lse_s = reinterpret_cast<const float*>(Qt + 2 * kTile);
  const float* D_s = lse_s + 64;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    f32x16_t sc, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sc[r] = 0.f;
      dp[r] = 0.f;
    }
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) {
      sc = mfma16<F>(to.frag(Qt, t, kk), kf[kk], sc);
      dp = mfma16<F>(to.frag(dOt, t, kk), to.frag(Vt, wave, kk), dp);
      // keeps the fragment reads next to their MFMAs: two waves per SIMD
      // hide the latency, and the register budget is 256
      if constexpr (HD == 128) __builtin_amdgcn_sched_barrier(0);
    }
    // lane holds key column kvrow; query rows t*32 + 8*(r/4) + 4*half + r%4
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int qlb = t * 32 + 8 * r4 + 4 * half;
      const float4 l4 = *reinterpret_cast<const float4*>(lse_s + qlb);
      const float4 d4 = *reinterpret_cast<const float4*>(D_s + qlb);
      const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
      const float dvv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * r4 + e;
        float p = __builtin_amdgcn_exp2f(fmaf(sc[r], c, -lv[e] * kLog2e));
        if constexpr (MASK) p = kvrow <= q0 + qlb + e ? p : 0.f;
        dp[r] = p * (dp[r] - dvv[e]);
        sc[r] = p;
      }
    }
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      const int ks = 2 * t + kh;
      const bf16x8_t pb = pack8<F>(sc, 8 * kh);
      const bf16x8_t dsb = pack8<F>(dp, 8 * kh);
#pragma unroll
      for (int i = 0; i < HD / 32; ++i) {
        dv[i] = mfma16<F>(to.frag_t(dOt, ks, i), pb, dv[i]);
        dk[i] = mfma16<F>(to.frag_t(Qt, ks, i), dsb, dk[i]);
        if constexpr (HD == 128) __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
}

template <int HD, typename F>
__global__ void __launch_bounds__(512) attn_bwd_dkdv_wide_kernel(AttnArgs a) {
  constexpr int BKV = 256, BQ = 64;
  constexpr int kTile = BQ * HD * 2;
  constexpr int kVTile = BKV * HD * 2;
  constexpr int kStage = 2 * kTile + 512;  // Q, dO, lse[64], delta[64]
  __shared__ __attribute__((aligned(1024))) char smem[kVTile + 2 * kStage];

  const int S = a.S, H = a.H, KV = a.KV, rep = H / KV;
  int kvb, b, g;
  key_block_coords(blockIdx.x, a.B, KV, kvb, b, g);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, l32 = lane & 31;
  TileOffsets<HD> to;
  to.init(lane);
  const int k0 = kvb * BKV, kw0 = k0 + 32 * wave;
  const int kvrow = kw0 + l32;
  const float c = a.scale * kLog2e;
  const char* Vt = smem;
  char* stages = smem + kVTile;

  {  // the V tile: 64-row quarters 2*(wave/4) and 2*(wave/4)+1
    const int quarter0 = 2 * (wave >> 2);
#pragma unroll
    for (int qq = 0; qq < 2; ++qq) {
      const int r0 = k0 + 64 * (quarter0 + qq);
      dma_tile_rows<HD>(a.v + ((int64_t)b * S + min(r0, S - 1)) * a.ldv + (int64_t)g * HD, a.ldv, S - min(r0, S - 1),
                        smem + (quarter0 + qq) * kTile, wave & 3, lane);
    }
  }
  bf16x8_t kf[HD / 16];
  {
    const int64_t r = (int64_t)b * S + min(kvrow, S - 1);
    const uint16_t* kp = a.k + r * a.ldk + (int64_t)g * HD + 8 * half;
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk)
      kf[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(kp + kk * 16));
  }
  f32x16_t dk[HD / 32], dv[HD / 32];
#pragma unroll
  for (int i = 0; i < HD / 32; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dk[i][r] = 0.f;
      dv[i][r] = 0.f;
    }

  const int qstart = (k0 / BQ) * BQ;
  const int nqs = (S - qstart) / BQ;
  const int nsteps = rep * nqs;
  auto open_step = [&](int step) {
    dma_barrier();  // this step's tiles (and the V tile) landed, last step's reads retired
    if (step + 1 < nsteps)
      dkdv8_issue<HD>(a, step + 1, nqs, qstart, b, g, rep, stages + ((step + 1) & 1) * kStage, wave, lane);
  };
  // Per query head, the 64-query blocks j = 0 .. nqs-1 (queries qstart + 64j
  // on) fall into three runs for this wave's keys kw0 .. kw0+31 (kw0 a
  // multiple of 32): blocks wholly before the keys (no work), blocks across
  // the diagonal (masked), blocks wholly after it (unmasked).  Every wave
  // opens every step, so the barriers match.
  const int rel = kw0 - qstart;  // 0 .. 224
  const int j_first = kw0 < S ? min(nqs, rel / BQ) : nqs;
  const int j_unmasked = kw0 < S ? min(nqs, (rel + 32 + BQ - 1) / BQ) : nqs;
  dkdv8_issue<HD>(a, 0, nqs, qstart, b, g, rep, stages, wave, lane);
  int step = 0;
  for (int hq = 0; hq < rep; ++hq) {
    int j = 0;
    for (; j < j_first; ++j, ++step) open_step(step);
    for (; j < j_unmasked; ++j, ++step) {
      open_step(step);
      dkdv_step<HD, true, F>(dk, dv, to, stages + (step & 1) * kStage, Vt, kf, c, qstart + j * BQ, kvrow, wave, half);
    }
    for (; j < nqs; ++j, ++step) {
      open_step(step);
      dkdv_step<HD, false, F>(dk, dv, to, stages + (step & 1) * kStage, Vt, kf, c, qstart + j * BQ, kvrow, wave, half);
    }
  }
  if (kvrow < S) {
    uint16_t* dkp = a.dk + ((int64_t)b * S + kvrow) * a.lddk + (int64_t)g * HD;
    uint16_t* dvp = a.dv + ((int64_t)b * S + kvrow) * a.lddv + (int64_t)g * HD;
    const bool rope = a.rcos != nullptr;
    store_grad_row<HD, F>(dkp, dk, a.scale, half, rope ? a.rcos + (int64_t)kvrow * HD : nullptr,
                       rope ? a.rsin + (int64_t)kvrow * HD : nullptr);
    store_grad_row<HD, F>(dvp, dv, 1.0f, half, nullptr, nullptr);
  }
}

// One 64-key step of the dQ kernel for this wave's 32 queries: S and dP, dS,
// then dQ += dS K.  MASK: the step holds this wave's diagonal, so keys past
// the query are dropped (the other steps carry no masking instructions).
template <int HD, bool MASK, typename F>
__device__ __forceinline__ void dq_step(f32x16_t (&dq)[HD / 32], const TileOffsets<HD>& to, const char* Kt,
                                        const bf16x8_t (&qf)[HD / 16], const bf16x8_t (&df)[HD / 16], float c, float nl2,
                                        float Dq, int k0, int qrow, int half) {
  constexpr int kTile = 64 * HD * 2;
  const char* Vt = Kt + kTile;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    f32x16_t st, dpt;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      st[r] = 0.f;
      dpt[r] = 0.f;
    }
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) {
      st = mfma16<F>(to.frag(Kt, t, kk), qf[kk], st);
      dpt = mfma16<F>(to.frag(Vt, t, kk), df[kk], dpt);
    }
    // the K^T fragments of the first 16 keys, read before dS is formed so
    // that the dQ MFMAs do not wait for LDS; the next 16 keys' during them
    bf16x8_t kt[2][HD / 32];
#pragma unroll
    for (int i = 0; i < HD / 32; ++i) kt[0][i] = to.frag_t(Kt, 2 * t, i);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float p = __builtin_amdgcn_exp2f(fmaf(st[r], c, nl2));
      if constexpr (MASK) {
        const int kv = k0 + t * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        p = kv <= qrow ? p : 0.f;
      }
      dpt[r] = p * (dpt[r] - Dq);
    }
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      if (kh == 0)
#pragma unroll
        for (int i = 0; i < HD / 32; ++i) kt[1][i] = to.frag_t(Kt, 2 * t + 1, i);
      const bf16x8_t dsb = pack8<F>(dpt, 8 * kh);
#pragma unroll
      for (int i = 0; i < HD / 32; ++i)
        dq[i] = mfma16<F>(kt[kh][i], dsb, dq[i]);
    }
  }
}

// dQ on tiles: 128 queries per workgroup, 64-key steps up to the diagonal.
// kDelta: delta = rowsum(dO * O) of the workgroup's queries is computed here
// (from the dO fragments held in registers and the same columns of O, a.o)
// and written to a.delta_w for the dK/dV kernel that runs next, instead of
// read from a.delta.
template <int HD, typename F, bool kDelta = false>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) attn_bwd_dq_tile_kernel(AttnArgs a) {
  constexpr int BQ = 128, BKV = 64;
  constexpr int kTile = BKV * HD * 2;
  constexpr int kStage = 2 * kTile;  // K, V
  __shared__ __attribute__((aligned(1024))) char smem[2 * kStage];

  const int S = a.S, H = a.H, KV = a.KV;
  const int nqb = (S + BQ - 1) / BQ;
  int qb, b, h;
  query_block_coords(blockIdx.x, nqb, a.B, H, KV, qb, b, h);
  const int g = h / (H / KV);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, l32 = lane & 31;
  TileOffsets<HD> to;
  to.init(lane);
  const int q0 = qb * BQ, qw0 = q0 + 32 * wave;
  const int qrow = qw0 + l32;
  const int qc = min(qrow, S - 1);
  const float c = a.scale * kLog2e;

  bf16x8_t qf[HD / 16], df[HD / 16];
  {
    const uint16_t* qp = a.q + ((int64_t)b * S + qc) * a.ldq + (int64_t)h * HD + 8 * half;
    const uint16_t* dp_ = a.dout + ((int64_t)b * S + qc) * a.lddo + (int64_t)h * HD + 8 * half;
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) {
      qf[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(qp + kk * 16));
      df[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(dp_ + kk * 16));
    }
  }
  const float nl2 = -a.lse[((int64_t)b * H + h) * S + qc] * kLog2e;
  float Dq;
  if constexpr (kDelta) {
    // each half of the wave holds half of the row's columns (8 of every 16)
    const uint16_t* op = a.o + ((int64_t)b * S + qc) * a.ldo + (int64_t)h * HD + 8 * half;
    float acc = 0.f;
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) {
      const uint4 ov = *reinterpret_cast<const uint4*>(op + kk * 16);
      const uint4 dv = __builtin_bit_cast(uint4, df[kk]);
      const uint32_t ow[4] = {ov.x, ov.y, ov.z, ov.w}, dw[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
      for (int k2 = 0; k2 < 4; ++k2) {
        acc = fmaf(F::to_f(ow[k2] & 0xffff), F::to_f(dw[k2] & 0xffff), acc);
        acc = fmaf(F::to_f(ow[k2] >> 16), F::to_f(dw[k2] >> 16), acc);
      }
    }
    Dq = sum_halves(acc);
    if (qrow < S && half == 0) a.delta_w[((int64_t)b * H + h) * S + qrow] = Dq;
  } else {
    Dq = a.delta[((int64_t)b * H + h) * S + qc];
  }
  f32x16_t dq[HD / 32];
#pragma unroll
  for (int i = 0; i < HD / 32; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[i][r] = 0.f;

  const int kv_end = min(S, q0 + BQ);
  const int kv_end_w = qw0 < S ? min(S, qw0 + 32) : 0;  // a wave past the sequence computes nothing
  const uint16_t* kbase = a.k + (int64_t)b * S * a.ldk + (int64_t)g * HD;
  const uint16_t* vbase = a.v + (int64_t)b * S * a.ldv + (int64_t)g * HD;
  const int nsteps = kv_end / BKV;

  auto open_step = [&](int it) {
    dma_barrier();  // this step's tiles landed (every wave's loads), last step's reads retired
    if (it + 1 < nsteps) {
      char* nxt = smem + ((it + 1) & 1) * kStage;
      dma_tile<HD>(kbase + (int64_t)(it + 1) * BKV * a.ldk, a.ldk, nxt, wave, lane);
      dma_tile<HD>(vbase + (int64_t)(it + 1) * BKV * a.ldv, a.ldv, nxt + kTile, wave, lane);
    }
  };
  // This wave's last step holds its diagonal (the only masked step); the
  // steps after it only join the barriers.
  const int last_w = kv_end_w > 0 ? (kv_end_w - 1) / BKV : -1;
  dma_tile<HD>(kbase, a.ldk, smem, wave, lane);
  dma_tile<HD>(vbase, a.ldv, smem + kTile, wave, lane);
  int it = 0;
  for (; it < last_w; ++it) {
    open_step(it);
    dq_step<HD, false, F>(dq, to, smem + (it & 1) * kStage, qf, df, c, nl2, Dq, it * BKV, qrow, half);
  }
  if (last_w >= 0) {
    open_step(it);
    dq_step<HD, true, F>(dq, to, smem + (it & 1) * kStage, qf, df, c, nl2, Dq, it * BKV, qrow, half);
    ++it;
  }
  for (; it < nsteps; ++it) open_step(it);
  if (qrow < S) {
    uint16_t* dqp = a.dq + ((int64_t)b * S + qrow) * a.lddq + (int64_t)h * HD;
    const bool rope = a.rcos != nullptr;
    store_grad_row<HD, F>(dqp, dq, a.scale, half, rope ? a.rcos + (int64_t)qrow * HD : nullptr,
                       rope ? a.rsin + (int64_t)qrow * HD : nullptr);
  }
}

// delta[b,h,s] = sum_d dO[b,s,h,d] * O[b,s,h,d]; one wave per (b, s, h) row.
template <typename T>
__global__ void __launch_bounds__(256) attn_delta_kernel(const T* __restrict__ o, int64_t ldo, const T* __restrict__ dout,
                                                          int64_t lddo, float* __restrict__ delta, int B, int S, int H,
                                                          int hd) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t total = (int64_t)B * S * H;
  if (row >= total) return;
  const int64_t bs = row / H;
  const int h = (int)(row - bs * H);
  const T* op = o + bs * ldo + (int64_t)h * hd;
  const T* dp = dout + bs * lddo + (int64_t)h * hd;
  float acc = 0.f;
  for (int d = lane; d < hd; d += 64) acc = fmaf(Elem<T>::load(op, d), Elem<T>::load(dp, d), acc);
  acc = wave_sum(acc);
  if (lane == 0) {
    const int64_t b = bs / S, s = bs - b * S;
    delta[(b * H + h) * S + s] = acc;
  }
}

// bf16 vector path: CPR = hd / 8 consecutive lanes share one (b, s, h) row,
// each loading 16 bytes of O and of dO (nontemporal: both are streamed
// once), so a workgroup reads 256 x 16 contiguous bytes of each; the row's
// partial sums meet through lane shuffles.  rows = B*S*H < 2^31.
template <int CPR>
__global__ void __launch_bounds__(256) attn_delta_vec_kernel(const uint16_t* __restrict__ o, int64_t ldo,
                                                              const uint16_t* __restrict__ dout, int64_t lddo,
                                                              float* __restrict__ delta, int S, int H, int rows) {
  typedef unsigned int v4u __attribute__((ext_vector_type(4)));
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int row = i / CPR, c = i % CPR;
  float acc = 0.f;
  if (row < rows) {
    const int bs = row / H, h = row - bs * H;
    const int64_t off = (int64_t)h * (CPR * 8) + c * 8;
    const v4u ov = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(o + bs * ldo + off));
    const v4u dv = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(dout + bs * lddo + off));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      acc = fmaf(bf2f(ov[k] & 0xffff), bf2f(dv[k] & 0xffff), acc);
      acc = fmaf(bf2f(ov[k] >> 16), bf2f(dv[k] >> 16), acc);
    }
  }
#pragma unroll
  for (int m = CPR / 2; m > 0; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (row < rows && c == 0) {
    const int bs = row / H, h = row - bs * H;
    const int b = bs / S, s = bs - b * S;
    delta[((int64_t)b * H + h) * S + s] = acc;
  }
}

// ---------------------------------------------------------------------------
// Generic path (any even head dim up to 256, bf16 or fp32): one wave per
// query row (forward, dQ) or key row (dK/dV), lanes split the head dim, fp32
// online softmax.  Used where the MFMA tiling does not apply.
// ---------------------------------------------------------------------------
template <typename T>
struct GenArgs {
  const T* q;
  const T* k;
  const T* v;
  int64_t ldq, ldk, ldv;
  T* o;
  int64_t ldo;
  float* lse;
  const T* dout;
  int64_t lddo;
  const float* delta;
  T* dq;
  T* dk;
  T* dv;
  int64_t lddq, lddk, lddv;
  int B, S, H, KV, hd;
  float scale;
  // explicit mask (SDPA's attn_mask; then no causal mask): kind 1 = bool
  // (bytes, nonzero keeps the score), 2 = fp32, 3 = bf16, 4 = fp16 (added to the
  // scaled score); element strides over [B, H, S(query), S(key)], 0 where
  // the mask broadcasts
  const void* mask;
  int mask_kind;
  int64_t msb, msh, msq, msk;
  // attention dropout (SDPA dropout_p): the probability of (b, h, query s,
  // key kv) is kept with scale 1/(1-p) when element ((b*H + h)*S + s)*S + kv
  // of the seed's stream is kept (lz_keep); drop_thresh 0 = no dropout
  uint32_t drop_thresh;
  float drop_scale;
  uint64_t drop_seed;
};

// Dropout factor of one attention probability (1 without dropout).
template <typename T>
__device__ __forceinline__ float drop_factor(const GenArgs<T>& a, int b, int h, int s, int kv) {
  if (a.drop_thresh == 0) return 1.0f;
  const uint64_t i = (((uint64_t)b * a.H + h) * a.S + s) * a.S + kv;
  return lz_keep(a.drop_seed, i, a.drop_thresh) ? a.drop_scale : 0.0f;
}

constexpr int kGenMax = 4;  // head dim up to 64 * kGenMax

// The scaled score of (b, h, query s, key kv) with the explicit mask applied:
// -inf where a bool mask is false, score + mask for a float mask.
template <typename T>
__device__ __forceinline__ float masked_score(const GenArgs<T>& a, float sc, int b, int h, int s, int kv) {
  const int64_t i = (int64_t)b * a.msb + (int64_t)h * a.msh + (int64_t)s * a.msq + (int64_t)kv * a.msk;
  if (a.mask_kind == 1) return static_cast<const uint8_t*>(a.mask)[i] ? sc : -INFINITY;
  if (a.mask_kind == 2) return sc + static_cast<const float*>(a.mask)[i];
  if (a.mask_kind == 3) return sc + bf2f(static_cast<const uint16_t*>(a.mask)[i]);
  return sc + h2f(static_cast<const uint16_t*>(a.mask)[i]);
}

template <typename T>
__global__ void __launch_bounds__(256) attn_fwd_generic_kernel(GenArgs<T> a) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t total = (int64_t)a.B * a.H * a.S;
  if (row >= total) return;
  const int s = (int)(row % a.S);
  const int64_t bh = row / a.S;
  const int h = (int)(bh % a.H), b = (int)(bh / a.H);
  const int g = h / (a.H / a.KV);
  const T* qp = a.q + ((int64_t)b * a.S + s) * a.ldq + (int64_t)h * a.hd;
  float qv[kGenMax], ov[kGenMax];
#pragma unroll
  for (int j = 0; j < kGenMax; ++j) {
    const int d = lane + 64 * j;
    qv[j] = d < a.hd ? Elem<T>::load(qp, d) : 0.f;
    ov[j] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int kv_last = a.mask_kind ? a.S - 1 : s;  // an explicit mask replaces the causal one
  for (int kv = 0; kv <= kv_last; ++kv) {
    const T* kp = a.k + ((int64_t)b * a.S + kv) * a.ldk + (int64_t)g * a.hd;
    const T* vp = a.v + ((int64_t)b * a.S + kv) * a.ldv + (int64_t)g * a.hd;
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < kGenMax; ++j) {
      const int d = lane + 64 * j;
      if (d < a.hd) dot = fmaf(qv[j], Elem<T>::load(kp, d), dot);
    }
    float sc = wave_sum(dot) * a.scale;
    if (a.mask_kind) {
      sc = masked_score(a, sc, b, h, s, kv);
      if (sc == -INFINITY) continue;  // contributes nothing (and keeps m finite once it is)
    }
    const float m_new = fmaxf(m, sc);
    const float corr = expf(m - m_new), p = expf(sc - m_new);
    l = l * corr + p;  // the normaliser sums the probabilities before dropout
    const float pz = p * drop_factor(a, b, h, s, kv);
#pragma unroll
    for (int j = 0; j < kGenMax; ++j) {
      const int d = lane + 64 * j;
      if (d < a.hd) ov[j] = ov[j] * corr + pz * Elem<T>::load(vp, d);
    }
    m = m_new;
  }
  T* op = a.o + ((int64_t)b * a.S + s) * a.ldo + (int64_t)h * a.hd;
#pragma unroll
  for (int j = 0; j < kGenMax; ++j) {
    const int d = lane + 64 * j;
    if (d < a.hd) Elem<T>::store(op, d, ov[j] / l);
  }
  if (lane == 0) a.lse[((int64_t)b * a.H + h) * a.S + s] = m + logf(l);
}

template <typename T>
__global__ void __launch_bounds__(256) attn_bwd_dq_generic_kernel(GenArgs<T> a) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t total = (int64_t)a.B * a.H * a.S;
  if (row >= total) return;
  const int s = (int)(row % a.S);
  const int64_t bh = row / a.S;
  const int h = (int)(bh % a.H), b = (int)(bh / a.H);
  const int g = h / (a.H / a.KV);
  const T* qp = a.q + ((int64_t)b * a.S + s) * a.ldq + (int64_t)h * a.hd;
  const T* dop = a.dout + ((int64_t)b * a.S + s) * a.lddo + (int64_t)h * a.hd;
  float qv[kGenMax], dov[kGenMax], acc[kGenMax];
#pragma unroll
  for (int j = 0; j < kGenMax; ++j) {
    const int d = lane + 64 * j;
    qv[j] = d < a.hd ? Elem<T>::load(qp, d) : 0.f;
    dov[j] = d < a.hd ? Elem<T>::load(dop, d) : 0.f;
    acc[j] = 0.f;
  }
  const float lse = a.lse[((int64_t)b * a.H + h) * a.S + s];
  const float D = a.delta[((int64_t)b * a.H + h) * a.S + s];
  const int kv_last = a.mask_kind ? a.S - 1 : s;
  for (int kv = 0; kv <= kv_last; ++kv) {
    const T* kp = a.k + ((int64_t)b * a.S + kv) * a.ldk + (int64_t)g * a.hd;
    const T* vp = a.v + ((int64_t)b * a.S + kv) * a.ldv + (int64_t)g * a.hd;
    float dot = 0.f, dpd = 0.f;
#pragma unroll
    for (int j = 0; j < kGenMax; ++j) {
      const int d = lane + 64 * j;
      if (d < a.hd) {
        dot = fmaf(qv[j], Elem<T>::load(kp, d), dot);
        dpd = fmaf(dov[j], Elem<T>::load(vp, d), dpd);
      }
    }
    float sc = wave_sum(dot) * a.scale;
    if (a.mask_kind) sc = masked_score(a, sc, b, h, s, kv);
    const float p = expf(sc - lse);
    // dL/dP = Z * dO.V for the dropped-out P; D = rowsum(dO * O) is unchanged
    const float ds = p * (drop_factor(a, b, h, s, kv) * wave_sum(dpd) - D);
#pragma unroll
    for (int j = 0; j < kGenMax; ++j) {
      const int d = lane + 64 * j;
      if (d < a.hd) acc[j] = fmaf(ds, Elem<T>::load(kp, d), acc[j]);
    }
  }
  T* dqp = a.dq + ((int64_t)b * a.S + s) * a.lddq + (int64_t)h * a.hd;
#pragma unroll
  for (int j = 0; j < kGenMax; ++j) {
    const int d = lane + 64 * j;
    if (d < a.hd) Elem<T>::store(dqp, d, acc[j] * a.scale);
  }
}

template <typename T>
__global__ void __launch_bounds__(256) attn_bwd_dkdv_generic_kernel(GenArgs<T> a) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t total = (int64_t)a.B * a.KV * a.S;
  if (row >= total) return;
  const int kv = (int)(row % a.S);
  const int64_t bg = row / a.S;
  const int g = (int)(bg % a.KV), b = (int)(bg / a.KV);
  const int rep = a.H / a.KV;
  const T* kp = a.k + ((int64_t)b * a.S + kv) * a.ldk + (int64_t)g * a.hd;
  const T* vp = a.v + ((int64_t)b * a.S + kv) * a.ldv + (int64_t)g * a.hd;
  float kvv[kGenMax], vvv[kGenMax], dka[kGenMax], dva[kGenMax];
#pragma unroll
  for (int j = 0; j < kGenMax; ++j) {
    const int d = lane + 64 * j;
    kvv[j] = d < a.hd ? Elem<T>::load(kp, d) : 0.f;
    vvv[j] = d < a.hd ? Elem<T>::load(vp, d) : 0.f;
    dka[j] = 0.f;
    dva[j] = 0.f;
  }
  for (int hq = 0; hq < rep; ++hq) {
    const int h = g * rep + hq;
    for (int s = a.mask_kind ? 0 : kv; s < a.S; ++s) {
      const T* qp = a.q + ((int64_t)b * a.S + s) * a.ldq + (int64_t)h * a.hd;
      const T* dop = a.dout + ((int64_t)b * a.S + s) * a.lddo + (int64_t)h * a.hd;
      float dot = 0.f, dpd = 0.f;
#pragma unroll
      for (int j = 0; j < kGenMax; ++j) {
        const int d = lane + 64 * j;
        if (d < a.hd) {
          dot = fmaf(Elem<T>::load(qp, d), kvv[j], dot);
          dpd = fmaf(Elem<T>::load(dop, d), vvv[j], dpd);
        }
      }
      const int64_t li = ((int64_t)b * a.H + h) * a.S + s;
      float sc = wave_sum(dot) * a.scale;
      if (a.mask_kind) sc = masked_score(a, sc, b, h, s, kv);
      const float p = expf(sc - a.lse[li]);
      const float z = drop_factor(a, b, h, s, kv);
      const float ds = p * (z * wave_sum(dpd) - a.delta[li]);
      const float pz = p * z;
#pragma unroll
      for (int j = 0; j < kGenMax; ++j) {
        const int d = lane + 64 * j;
        if (d < a.hd) {
          dva[j] = fmaf(pz, Elem<T>::load(dop, d), dva[j]);
          dka[j] = fmaf(ds, Elem<T>::load(qp, d), dka[j]);
        }
      }
    }
  }
  T* dkp = a.dk + ((int64_t)b * a.S + kv) * a.lddk + (int64_t)g * a.hd;
  T* dvp = a.dv + ((int64_t)b * a.S + kv) * a.lddv + (int64_t)g * a.hd;
#pragma unroll
  for (int j = 0; j < kGenMax; ++j) {
    const int d = lane + 64 * j;
    if (d < a.hd) {
      Elem<T>::store(dkp, d, dka[j] * a.scale);
      Elem<T>::store(dvp, d, dva[j]);
    }
  }
}

// ---------------------------------------------------------------------------
// Small head dims (16, 32): four lanes (a quad) per query row (forward, dQ)
// or key row (dK/dV), each holding a quarter of that row, its accumulators
// and the row's running softmax in registers; a workgroup of four waves owns
// 64 rows.  The other side's rows pass through LDS 64 at a time as fp32
// (written by consecutive threads, read by the 16 quads of a wave at four
// distinct addresses).  Dot products are summed over the quad with two DPP
// steps, which give all four lanes the same bits.
// ---------------------------------------------------------------------------

// rows [row0, row0 + n) of base[., ld] (columns 0 .. HD) into dst[64][HD] by
// 256 threads; rows from n on are zero.  Every load is unconditional (rows
// past n re-read row n-1), so they all issue before the first wait.
template <typename T, int HD>
__device__ __forceinline__ void stage_rows(float* dst, const T* base, int64_t ld, int64_t row0, int n, int tid) {
  constexpr int kPass = 64 * HD / 256;
  float x[kPass];
#pragma unroll
  for (int i = 0; i < kPass; ++i) {
    const int e = tid + 256 * i;
    const int r = min(e / HD, n - 1), d = e % HD;
    x[i] = Elem<T>::load(base + (row0 + r) * ld, d);
  }
#pragma unroll
  for (int i = 0; i < kPass; ++i) {
    const int e = tid + 256 * i;
    dst[e] = e / HD < n ? x[i] : 0.f;
  }
}

// DL values of a row from column c0 as fp32; rows the caller does not own
// read as zero
template <typename T, int DL>
__device__ __forceinline__ void load_part(float (&x)[DL], const T* p, bool own) {
#pragma unroll
  for (int d = 0; d < DL; ++d) x[d] = Elem<T>::load(p, d);
#pragma unroll
  for (int d = 0; d < DL; ++d) x[d] = own ? x[d] : 0.f;
}

// sum over the four lanes of a quad (quad_perm [1,0,3,2] then [2,3,0,1])
__device__ __forceinline__ float quad_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, true));
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, true));
  return x;
}

template <int DL>
__device__ __forceinline__ float dot_part(const float (&x)[DL], const float* row) {
  const float4* r4 = reinterpret_cast<const float4*>(row);
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < DL / 4; ++i) {
    const float4 t = r4[i];
    acc = fmaf(x[4 * i], t.x, acc);
    acc = fmaf(x[4 * i + 1], t.y, acc);
    acc = fmaf(x[4 * i + 2], t.z, acc);
    acc = fmaf(x[4 * i + 3], t.w, acc);
  }
  return acc;
}

// acc = acc * c + p * row
template <int DL>
__device__ __forceinline__ void axpby_part(float (&acc)[DL], float c, float p, const float* row) {
  const float4* r4 = reinterpret_cast<const float4*>(row);
#pragma unroll
  for (int i = 0; i < DL / 4; ++i) {
    const float4 t = r4[i];
    acc[4 * i] = fmaf(p, t.x, acc[4 * i] * c);
    acc[4 * i + 1] = fmaf(p, t.y, acc[4 * i + 1] * c);
    acc[4 * i + 2] = fmaf(p, t.z, acc[4 * i + 2] * c);
    acc[4 * i + 3] = fmaf(p, t.w, acc[4 * i + 3] * c);
  }
}

// grid: B * H * ceil(S / 64) workgroups of 256, query block fastest
template <typename T, int HD>
__global__ void __launch_bounds__(256) attn_fwd_quad_kernel(GenArgs<T> a) {
  constexpr int DL = HD / 4;
  __shared__ __attribute__((aligned(16))) float ks[64 * HD];
  __shared__ __attribute__((aligned(16))) float vs[64 * HD];
  const int tid = threadIdx.x, qd = tid & 3, rl = tid >> 2;
  const int nqb = (a.S + 63) / 64;
  const int qb = (int)(blockIdx.x % nqb);
  const int64_t bh = blockIdx.x / nqb;
  const int h = (int)(bh % a.H), b = (int)(bh / a.H);
  const int g = h / (a.H / a.KV);
  const int s = qb * 64 + rl;
  const bool valid = s < a.S;
  float q[DL], o[DL];
  load_part<T, DL>(q, a.q + ((int64_t)b * a.S + (valid ? s : 0)) * a.ldq + (int64_t)h * HD + qd * DL, valid);
#pragma unroll
  for (int d = 0; d < DL; ++d) o[d] = 0.f;
  const T* kb = a.k + (int64_t)b * a.S * a.ldk + (int64_t)g * HD;
  const T* vb = a.v + (int64_t)b * a.S * a.ldv + (int64_t)g * HD;
  const int kv_end = min(a.S, qb * 64 + 64);
  const int last = valid ? s : -1;  // causal: keys 0 .. s
  float m = -INFINITY, l = 0.f;
  for (int c0 = 0; c0 < kv_end; c0 += 64) {
    const int n = min(64, kv_end - c0);
    __syncthreads();  // the previous chunk's reads are done
    stage_rows<T, HD>(ks, kb, a.ldk, c0, n, tid);
    stage_rows<T, HD>(vs, vb, a.ldv, c0, n, tid);
    __syncthreads();
    const int jn = min(n, last - c0 + 1);  // the same for the four lanes of a row
    for (int j = 0; j < jn; ++j) {
      const float sc = quad_sum(dot_part<DL>(q, ks + j * HD + qd * DL)) * a.scale;
      const float m_new = fmaxf(m, sc);
      const float corr = expf(m - m_new), p = expf(sc - m_new);
      l = l * corr + p;
      axpby_part<DL>(o, corr, p, vs + j * HD + qd * DL);
      m = m_new;
    }
  }
  if (valid) {
    T* op = a.o + ((int64_t)b * a.S + s) * a.ldo + (int64_t)h * HD + qd * DL;
    const float inv = 1.f / l;
#pragma unroll
    for (int d = 0; d < DL; ++d) Elem<T>::store(op, d, o[d] * inv);
    if (qd == 0) a.lse[((int64_t)b * a.H + h) * a.S + s] = m + logf(l);
  }
}

template <typename T, int HD>
__global__ void __launch_bounds__(256) attn_bwd_dq_quad_kernel(GenArgs<T> a) {
  constexpr int DL = HD / 4;
  __shared__ __attribute__((aligned(16))) float ks[64 * HD];
  __shared__ __attribute__((aligned(16))) float vs[64 * HD];
  const int tid = threadIdx.x, qd = tid & 3, rl = tid >> 2;
  const int nqb = (a.S + 63) / 64;
  const int qb = (int)(blockIdx.x % nqb);
  const int64_t bh = blockIdx.x / nqb;
  const int h = (int)(bh % a.H), b = (int)(bh / a.H);
  const int g = h / (a.H / a.KV);
  const int s = qb * 64 + rl;
  const bool valid = s < a.S;
  const int64_t row = (int64_t)b * a.S + (valid ? s : 0);
  float q[DL], dov[DL], acc[DL];
  load_part<T, DL>(q, a.q + row * a.ldq + (int64_t)h * HD + qd * DL, valid);
  load_part<T, DL>(dov, a.dout + row * a.lddo + (int64_t)h * HD + qd * DL, valid);
#pragma unroll
  for (int d = 0; d < DL; ++d) acc[d] = 0.f;
  const int64_t li = ((int64_t)b * a.H + h) * a.S + (valid ? s : 0);
  const float lse = a.lse[li], D = a.delta[li];
  const T* kb = a.k + (int64_t)b * a.S * a.ldk + (int64_t)g * HD;
  const T* vb = a.v + (int64_t)b * a.S * a.ldv + (int64_t)g * HD;
  const int kv_end = min(a.S, qb * 64 + 64);
  const int last = valid ? s : -1;
  for (int c0 = 0; c0 < kv_end; c0 += 64) {
    const int n = min(64, kv_end - c0);
    __syncthreads();
    stage_rows<T, HD>(ks, kb, a.ldk, c0, n, tid);
    stage_rows<T, HD>(vs, vb, a.ldv, c0, n, tid);
    __syncthreads();
    const int jn = min(n, last - c0 + 1);
    for (int j = 0; j < jn; ++j) {
      const float* kr = ks + j * HD + qd * DL;
      const float p = expf(quad_sum(dot_part<DL>(q, kr)) * a.scale - lse);
      const float ds = p * (quad_sum(dot_part<DL>(dov, vs + j * HD + qd * DL)) - D);
      axpby_part<DL>(acc, 1.f, ds, kr);
    }
  }
  if (valid) {
    T* dqp = a.dq + ((int64_t)b * a.S + s) * a.lddq + (int64_t)h * HD + qd * DL;
#pragma unroll
    for (int d = 0; d < DL; ++d) Elem<T>::store(dqp, d, acc[d] * a.scale);
  }
}

// grid: B * KV * ceil(S / 64) workgroups of 256; a quad owns one key row and
// sums over the queries of every head in its group
template <typename T, int HD>
__global__ void __launch_bounds__(256) attn_bwd_dkdv_quad_kernel(GenArgs<T> a) {
  constexpr int DL = HD / 4;
  __shared__ __attribute__((aligned(16))) float qs[64 * HD];
  __shared__ __attribute__((aligned(16))) float dos[64 * HD];
  __shared__ float ls[64], dl[64];
  const int tid = threadIdx.x, qd = tid & 3, rl = tid >> 2;
  const int nkb = (a.S + 63) / 64;
  const int kbk = (int)(blockIdx.x % nkb);
  const int64_t bg = blockIdx.x / nkb;
  const int g = (int)(bg % a.KV), b = (int)(bg / a.KV);
  const int rep = a.H / a.KV;
  const int kv = kbk * 64 + rl;
  const bool valid = kv < a.S;
  const int64_t row = (int64_t)b * a.S + (valid ? kv : 0);
  float kr[DL], vr[DL], dk[DL], dv[DL];
  load_part<T, DL>(kr, a.k + row * a.ldk + (int64_t)g * HD + qd * DL, valid);
  load_part<T, DL>(vr, a.v + row * a.ldv + (int64_t)g * HD + qd * DL, valid);
#pragma unroll
  for (int d = 0; d < DL; ++d) {
    dk[d] = 0.f;
    dv[d] = 0.f;
  }
  const int first = valid ? kv : a.S;  // causal: queries kv .. S-1
  for (int hq = 0; hq < rep; ++hq) {
    const int h = g * rep + hq;
    const T* qb = a.q + (int64_t)b * a.S * a.ldq + (int64_t)h * HD;
    const T* dob = a.dout + (int64_t)b * a.S * a.lddo + (int64_t)h * HD;
    const int64_t li0 = ((int64_t)b * a.H + h) * a.S;
    for (int c0 = kbk * 64; c0 < a.S; c0 += 64) {
      const int n = min(64, a.S - c0);
      __syncthreads();
      stage_rows<T, HD>(qs, qb, a.ldq, c0, n, tid);
      stage_rows<T, HD>(dos, dob, a.lddo, c0, n, tid);
      if (tid < 64) {
        const int lr = min(tid, n - 1);
        const float lv = a.lse[li0 + c0 + lr], dvv = a.delta[li0 + c0 + lr];
        ls[tid] = lv;
        dl[tid] = dvv;
      }
      __syncthreads();
      for (int j = max(0, first - c0); j < n; ++j) {
        const float* qr = qs + j * HD + qd * DL;
        const float* dr = dos + j * HD + qd * DL;
        const float p = expf(quad_sum(dot_part<DL>(kr, qr)) * a.scale - ls[j]);
        const float ds = p * (quad_sum(dot_part<DL>(vr, dr)) - dl[j]);
        axpby_part<DL>(dv, 1.f, p, dr);
        axpby_part<DL>(dk, 1.f, ds, qr);
      }
    }
  }
  if (valid) {
    T* dkp = a.dk + row * a.lddk + (int64_t)g * HD + qd * DL;
    T* dvp = a.dv + row * a.lddv + (int64_t)g * HD + qd * DL;
#pragma unroll
    for (int d = 0; d < DL; ++d) {
      Elem<T>::store(dkp, d, dk[d] * a.scale);
      Elem<T>::store(dvp, d, dv[d]);
    }
  }
}

template <typename T>
void launch_fwd_small(const GenArgs<T>& a, hipStream_t s) {
  const unsigned grid = (unsigned)((int64_t)a.B * a.H * ((a.S + 63) / 64));
  if (a.hd == 16) attn_fwd_quad_kernel<T, 16><<<grid, 256, 0, s>>>(a);
  else attn_fwd_quad_kernel<T, 32><<<grid, 256, 0, s>>>(a);
}

template <typename T>
void launch_bwd_small(const GenArgs<T>& a, hipStream_t s) {
  const unsigned grid_q = (unsigned)((int64_t)a.B * a.H * ((a.S + 63) / 64));
  const unsigned grid_kv = (unsigned)((int64_t)a.B * a.KV * ((a.S + 63) / 64));
  if (a.hd == 16) {
    attn_bwd_dq_quad_kernel<T, 16><<<grid_q, 256, 0, s>>>(a);
    attn_bwd_dkdv_quad_kernel<T, 16><<<grid_kv, 256, 0, s>>>(a);
  } else {
    attn_bwd_dq_quad_kernel<T, 32><<<grid_q, 256, 0, s>>>(a);
    attn_bwd_dkdv_quad_kernel<T, 32><<<grid_kv, 256, 0, s>>>(a);
  }
}

// The tile loads address a tile's rows by 32-bit byte offsets from its first
// row: row strides below 2^22 elements keep a 64-row tile below 2^31 bytes.
constexpr int64_t kMaxTileLd = 1ll << 22;

bool strides_ok(int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo) {
  return ldq % 8 == 0 && ldk % 8 == 0 && ldv % 8 == 0 && ldo % 4 == 0 && ldq < kMaxTileLd && ldk < kMaxTileLd &&
         ldv < kMaxTileLd && ldo < kMaxTileLd;
}

bool mfma_ok(int dtype, int64_t hd, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo, const void* q, const void* k,
             const void* v, const void* o) {
  return (dtype == LZ_BF16 || dtype == LZ_F16) && (hd == 64 || hd == 128) && strides_ok(ldq, ldk, ldv, ldo) &&
         lz_aligned16(q) && lz_aligned16(k) && lz_aligned16(v) && (reinterpret_cast<uintptr_t>(o) & 7) == 0;
}

int check_shape(int64_t B, int64_t S, int64_t H, int64_t KV, int64_t hd) {
  LZ_REQUIRE(B > 0 && S > 0 && H > 0 && KV > 0 && hd > 0, "attention: bad shape");
  LZ_REQUIRE(H % KV == 0, "attention: H (%lld) must be a multiple of KV (%lld)", (long long)H, (long long)KV);
  LZ_REQUIRE(hd <= 64 * kGenMax, "attention: head dim %lld > %d", (long long)hd, 64 * kGenMax);
  LZ_REQUIRE(B * H * lz_cdiv(S, 64) < (1ll << 31) && S < (1 << 30), "attention: problem too large");
  return LZ_OK;
}

}  // namespace

// Which path lz_attn_fwd/bwd take for these arguments: 2 = MFMA on LDS tiles
// (S a multiple of 64; no transposed buffers), 1 = MFMA with the transposed
// operand buffers (V^T for the forward; Q^T, K^T, dO^T for the backward),
// 0 = generic.  fp16 takes the tile path or the generic one.
LZ_EXPORT int lz_attn_path(int dtype, int64_t S, int64_t hd, int64_t ldq, int64_t ldk, int64_t ldv, int64_t ldo) {
  const bool mfma = (dtype == LZ_BF16 || (dtype == LZ_F16 && S % 64 == 0)) && (hd == 64 || hd == 128) &&
                    strides_ok(ldq, ldk, ldv, ldo);
  return mfma ? (S % 64 == 0 ? 2 : 1) : 0;
}

// Forward.  vt: V^T [B,KV,hd,S] (needed on the MFMA path only).
LZ_EXPORT int lz_attn_fwd(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                          const void* vt, void* o, int64_t ldo, float* lse, int64_t B, int64_t S, int64_t H, int64_t KV,
                          int64_t hd, float scale, int dtype, void* stream) {
  int rc = check_shape(B, S, H, KV, hd);
  if (rc) return rc;
  LZ_REQUIRE(q && k && v && o && lse, "lz_attn_fwd: null pointer");
  hipStream_t s = lz_stream(stream);
  if (mfma_ok(dtype, hd, ldq, ldk, ldv, ldo, q, k, v, o) && S % 64 == 0) {
    AttnArgs a{};
    a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
    a.ldq = ldq; a.ldk = ldk; a.ldv = ldv;
    a.o = (uint16_t*)o; a.ldo = ldo; a.lse = lse;
    a.B = (int)B; a.S = (int)S; a.H = (int)H; a.KV = (int)KV; a.scale = scale;
    const unsigned grid = (unsigned)(lz_cdiv(S, 128) * B * H);
    if (dtype == LZ_F16) {
      if (hd == 128) attn_fwd_tile_kernel<128, FmtF16><<<grid, 256, 0, s>>>(a);
      else attn_fwd_tile_kernel<64, FmtF16><<<grid, 256, 0, s>>>(a);
    } else {
      if (hd == 128) attn_fwd_tile_kernel<128, FmtBF16><<<grid, 256, 0, s>>>(a);
      else attn_fwd_tile_kernel<64, FmtBF16><<<grid, 256, 0, s>>>(a);
    }
    return lz_check_launch("lz_attn_fwd");
  }
  if (dtype == LZ_BF16 && mfma_ok(dtype, hd, ldq, ldk, ldv, ldo, q, k, v, o)) {
    LZ_REQUIRE(vt && lz_aligned16(vt), "lz_attn_fwd: MFMA path needs an aligned V^T buffer");
    AttnArgs a{};
    a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
    a.ldq = ldq; a.ldk = ldk; a.ldv = ldv;
    a.o = (uint16_t*)o; a.ldo = ldo; a.lse = lse; a.vt = (const uint16_t*)vt;
    a.B = (int)B; a.S = (int)S; a.H = (int)H; a.KV = (int)KV; a.scale = scale;
    const unsigned grid = (unsigned)(lz_cdiv(S, 128) * B * H);
    if (hd == 128) attn_fwd_kernel<128><<<grid, 256, 0, s>>>(a);
    else attn_fwd_kernel<64><<<grid, 256, 0, s>>>(a);
    return lz_check_launch("lz_attn_fwd");
  }
  const unsigned grid = (unsigned)lz_cdiv(B * H * S, 4);
  if (dtype == LZ_BF16) {
    GenArgs<uint16_t> a{};
    a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
    a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.o = (uint16_t*)o; a.ldo = ldo; a.lse = lse;
    a.B = (int)B; a.S = (int)S; a.H = (int)H; a.KV = (int)KV; a.hd = (int)hd; a.scale = scale;
    if (hd == 16 || hd == 32) launch_fwd_small(a, s);
    else attn_fwd_generic_kernel<uint16_t><<<grid, 256, 0, s>>>(a);
  } else if (dtype == LZ_F16) {
    GenArgs<_Float16> a{};
    a.q = (const _Float16*)q; a.k = (const _Float16*)k; a.v = (const _Float16*)v;
    a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.o = (_Float16*)o; a.ldo = ldo; a.lse = lse;
    a.B = (int)B; a.S = (int)S; a.H = (int)H; a.KV = (int)KV; a.hd = (int)hd; a.scale = scale;
    if (hd == 16 || hd == 32) launch_fwd_small(a, s);
    else attn_fwd_generic_kernel<_Float16><<<grid, 256, 0, s>>>(a);
  } else if (dtype == LZ_F32) {
    GenArgs<float> a{};
    a.q = (const float*)q; a.k = (const float*)k; a.v = (const float*)v;
    a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.o = (float*)o; a.ldo = ldo; a.lse = lse;
    a.B = (int)B; a.S = (int)S; a.H = (int)H; a.KV = (int)KV; a.hd = (int)hd; a.scale = scale;
    if (hd == 16 || hd == 32) launch_fwd_small(a, s);
    else attn_fwd_generic_kernel<float><<<grid, 256, 0, s>>>(a);
  } else {
    return lz_set_error(LZ_EINVAL, "lz_attn_fwd: bad dtype %d", dtype);
  }
  return lz_check_launch("lz_attn_fwd(generic)");
}

LZ_EXPORT int lz_attn_delta(const void* o, int64_t ldo, const void* dout, int64_t lddo, float* delta, int64_t B, int64_t S,
                            int64_t H, int64_t hd, int dtype, void* stream) {
  LZ_REQUIRE(B > 0 && S > 0 && H > 0 && hd > 0 && delta, "lz_attn_delta: bad arguments");
  const unsigned grid = (unsigned)lz_cdiv(B * S * H, 4);
  hipStream_t s = lz_stream(stream);
  const int64_t rows = B * S * H;
  const bool vec = dtype == LZ_BF16 && (hd == 32 || hd == 64 || hd == 128 || hd == 256) && lz_aligned16(o) &&
                   lz_aligned16(dout) && ldo % 8 == 0 && lddo % 8 == 0 && rows * (hd / 8) < (1ll << 31);
  if (vec) {
    const unsigned vgrid = (unsigned)lz_cdiv(rows * (hd / 8), 256);
    const uint16_t *o16 = (const uint16_t*)o, *d16 = (const uint16_t*)dout;
    if (hd == 32) attn_delta_vec_kernel<4><<<vgrid, 256, 0, s>>>(o16, ldo, d16, lddo, delta, (int)S, (int)H, (int)rows);
    else if (hd == 64) attn_delta_vec_kernel<8><<<vgrid, 256, 0, s>>>(o16, ldo, d16, lddo, delta, (int)S, (int)H, (int)rows);
    else if (hd == 128) attn_delta_vec_kernel<16><<<vgrid, 256, 0, s>>>(o16, ldo, d16, lddo, delta, (int)S, (int)H, (int)rows);
    else attn_delta_vec_kernel<32><<<vgrid, 256, 0, s>>>(o16, ldo, d16, lddo, delta, (int)S, (int)H, (int)rows);
  } else if (dtype == LZ_BF16)
    attn_delta_kernel<uint16_t><<<grid, 256, 0, s>>>((const uint16_t*)o, ldo, (const uint16_t*)dout, lddo, delta, (int)B, (int)S, (int)H, (int)hd);
  else if (dtype == LZ_F32)
    attn_delta_kernel<float><<<grid, 256, 0, s>>>((const float*)o, ldo, (const float*)dout, lddo, delta, (int)B, (int)S, (int)H, (int)hd);
  else if (dtype == LZ_F16)
    attn_delta_kernel<_Float16><<<grid, 256, 0, s>>>((const _Float16*)o, ldo, (const _Float16*)dout, lddo, delta, (int)B, (int)S, (int)H, (int)hd);
  else
    return lz_set_error(LZ_EINVAL, "lz_attn_delta: bad dtype %d", dtype);
  return lz_check_launch("lz_attn_delta");
}

LZ_EXPORT int lz_rope(void* x, int dtype, int64_t ld, int64_t rows, int64_t seq, int64_t nheads, int64_t hd,
                      const void* cos_t, const void* sin_t, int64_t pos_offset, int backward, void* stream);

namespace {

int attn_bwd_impl(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv, const void* dout,
                  int64_t lddo, const float* lse, const float* delta, const void* qt, const void* kt, const void* dot,
                  void* dq, int64_t lddq, void* dk, int64_t lddk, void* dv, int64_t lddv, int64_t B, int64_t S,
                  int64_t H, int64_t KV, int64_t hd, float scale, const void* rope_cos, const void* rope_sin,
                  int dtype, hipStream_t s, bool& rope_done, const void* o = nullptr, int64_t ldo = 0,
                  float* delta_w = nullptr);

}  // namespace

// Backward.  On the MFMA path qt [B,H,hd,S], kt [B,KV,hd,S] and dot [B,H,hd,S]
// are required; delta comes from lz_attn_delta.  dq/dk/dv are written (not
// accumulated).  rope_cos/rope_sin (both or neither; tables [>= S, hd] in the
// activation dtype, row = position, as lz_rope takes): dq and dk come back
// as the gradients of q and k before RoPE, i.e. with lz_rope's backward
// already applied (in the bf16 MFMA kernels' epilogue, otherwise by lz_rope
// after them).
LZ_EXPORT int lz_attn_bwd(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                          const void* dout, int64_t lddo, const float* lse, const float* delta, const void* qt,
                          const void* kt, const void* dot, void* dq, int64_t lddq, void* dk, int64_t lddk, void* dv,
                          int64_t lddv, int64_t B, int64_t S, int64_t H, int64_t KV, int64_t hd, float scale,
                          const void* rope_cos, const void* rope_sin, int dtype, void* stream) {
  int rc = check_shape(B, S, H, KV, hd);
  if (rc) return rc;
  LZ_REQUIRE(q && k && v && dout && lse && delta && dq && dk && dv, "lz_attn_bwd: null pointer");
  LZ_REQUIRE((rope_cos == nullptr) == (rope_sin == nullptr), "lz_attn_bwd: give both RoPE tables or neither");
  LZ_REQUIRE(rope_cos == nullptr || (hd % 2 == 0 && ((reinterpret_cast<uintptr_t>(rope_cos) |
                                                        reinterpret_cast<uintptr_t>(rope_sin)) & 7) == 0),
             "lz_attn_bwd: RoPE needs an even head dim and 8-byte aligned tables");
  hipStream_t s = lz_stream(stream);
  bool rope_done = false;
  rc = attn_bwd_impl(q, ldq, k, ldk, v, ldv, dout, lddo, lse, delta, qt, kt, dot, dq, lddq, dk, lddk, dv, lddv, B, S,
                     H, KV, hd, scale, rope_cos, rope_sin, dtype, s, rope_done);
  if (rc || rope_cos == nullptr || rope_done) return rc;
  rc = lz_rope(dq, dtype, lddq, B * S, S, H, hd, rope_cos, rope_sin, 0, 1, stream);
  if (rc) return rc;
  return lz_rope(dk, dtype, lddk, B * S, S, KV, hd, rope_cos, rope_sin, 0, 1, stream);
}

// lz_attn_delta + lz_attn_bwd in one call for the LDS-tile kernels
// (lz_attn_path 2): the dQ kernel computes delta = rowsum(dO * O) from the
// dO rows it loads anyway and writes it to `delta` ([B, H, S] fp32, output),
// then the dK/dV kernel reads it.  Other shapes are refused.
LZ_EXPORT int lz_attn_bwd_with_o(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                                 const void* o, int64_t ldo, const void* dout, int64_t lddo, const float* lse,
                                 float* delta, void* dq, int64_t lddq, void* dk, int64_t lddk, void* dv, int64_t lddv,
                                 int64_t B, int64_t S, int64_t H, int64_t KV, int64_t hd, float scale,
                                 const void* rope_cos, const void* rope_sin, int dtype, void* stream) {
  int rc = check_shape(B, S, H, KV, hd);
  if (rc) return rc;
  LZ_REQUIRE(q && k && v && o && dout && lse && delta && dq && dk && dv, "lz_attn_bwd_with_o: null pointer");
  LZ_REQUIRE(lz_aligned16(o) && ldo % 8 == 0 && ldo >= H * hd, "lz_attn_bwd_with_o: O rows must be 16-byte aligned");
  LZ_REQUIRE((rope_cos == nullptr) == (rope_sin == nullptr), "lz_attn_bwd_with_o: give both RoPE tables or neither");
  LZ_REQUIRE(rope_cos == nullptr || (hd % 2 == 0 && ((reinterpret_cast<uintptr_t>(rope_cos) |
                                                        reinterpret_cast<uintptr_t>(rope_sin)) & 7) == 0),
             "lz_attn_bwd_with_o: RoPE needs an even head dim and 8-byte aligned tables");
  bool rope_done = false;
  return attn_bwd_impl(q, ldq, k, ldk, v, ldv, dout, lddo, lse, delta, nullptr, nullptr, nullptr, dq, lddq, dk, lddk,
                       dv, lddv, B, S, H, KV, hd, scale, rope_cos, rope_sin, dtype, lz_stream(stream), rope_done, o,
                       ldo, delta);
}

namespace {

int attn_bwd_impl(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv, const void* dout,
                  int64_t lddo, const float* lse, const float* delta, const void* qt, const void* kt, const void* dot,
                  void* dq, int64_t lddq, void* dk, int64_t lddk, void* dv, int64_t lddv, int64_t B, int64_t S,
                  int64_t H, int64_t KV, int64_t hd, float scale, const void* rope_cos, const void* rope_sin,
                  int dtype, hipStream_t s, bool& rope_done, const void* o, int64_t ldo, float* delta_w) {
  const bool mfma = mfma_ok(dtype, hd, ldq, ldk, ldv, lddo, q, k, v, dout) && lddq % 4 == 0 && lddk % 4 == 0 &&
                    lddv % 4 == 0;
  LZ_REQUIRE(delta_w == nullptr || (mfma && S % 64 == 0),
             "lz_attn_bwd_with_o: this shape takes the other kernels (use lz_attn_delta + lz_attn_bwd)");
  if (mfma && S % 64 == 0) {
    AttnArgs a{};
    a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
    a.ldq = ldq; a.ldk = ldk; a.ldv = ldv;
    a.lse = const_cast<float*>(lse);
    a.dout = (const uint16_t*)dout; a.lddo = lddo; a.delta = delta;
    a.dq = (uint16_t*)dq; a.dk = (uint16_t*)dk; a.dv = (uint16_t*)dv;
    a.lddq = lddq; a.lddk = lddk; a.lddv = lddv;
    a.rcos = (const uint16_t*)rope_cos; a.rsin = (const uint16_t*)rope_sin;
    rope_done = true;
    a.B = (int)B; a.S = (int)S; a.H = (int)H; a.KV = (int)KV; a.scale = scale;
    const unsigned grid_kv = (unsigned)(lz_cdiv(S, 256) * B * KV);
    const unsigned grid_q = (unsigned)(lz_cdiv(S, 128) * B * H);
    if (delta_w) {
      // the dQ pass computes delta (rowsum(dO * O)) and runs first; dK/dV reads it
      a.o = (uint16_t*)const_cast<void*>(o);
      a.ldo = ldo;
      a.delta_w = delta_w;
      a.delta = delta_w;
      if (dtype == LZ_F16) {
        if (hd == 128) attn_bwd_dq_tile_kernel<128, FmtF16, true><<<grid_q, 256, 0, s>>>(a);
        else attn_bwd_dq_tile_kernel<64, FmtF16, true><<<grid_q, 256, 0, s>>>(a);
      } else {
        if (hd == 128) attn_bwd_dq_tile_kernel<128, FmtBF16, true><<<grid_q, 256, 0, s>>>(a);
        else attn_bwd_dq_tile_kernel<64, FmtBF16, true><<<grid_q, 256, 0, s>>>(a);
      }
      const int rc = lz_check_launch("lz_attn_bwd_with_o");
      if (rc) return rc;
      if (dtype == LZ_F16) {
        if (hd == 128) attn_bwd_dkdv_wide_kernel<128, FmtF16><<<grid_kv, 512, 0, s>>>(a);
        else attn_bwd_dkdv_wide_kernel<64, FmtF16><<<grid_kv, 512, 0, s>>>(a);
      } else {
        if (hd == 128) attn_bwd_dkdv_wide_kernel<128, FmtBF16><<<grid_kv, 512, 0, s>>>(a);
        else attn_bwd_dkdv_wide_kernel<64, FmtBF16><<<grid_kv, 512, 0, s>>>(a);
      }
      return lz_check_launch("lz_attn_bwd_with_o");
    }
    if (dtype == LZ_F16) {
      if (hd == 128) {
        attn_bwd_dkdv_wide_kernel<128, FmtF16><<<grid_kv, 512, 0, s>>>(a);
        attn_bwd_dq_tile_kernel<128, FmtF16><<<grid_q, 256, 0, s>>>(a);
      } else {
        attn_bwd_dkdv_wide_kernel<64, FmtF16><<<grid_kv, 512, 0, s>>>(a);
        attn_bwd_dq_tile_kernel<64, FmtF16><<<grid_q, 256, 0, s>>>(a);
      }
    } else if (hd == 128) {
      attn_bwd_dkdv_wide_kernel<128, FmtBF16><<<grid_kv, 512, 0, s>>>(a);
      attn_bwd_dq_tile_kernel<128, FmtBF16><<<grid_q, 256, 0, s>>>(a);
    } else {
      attn_bwd_dkdv_wide_kernel<64, FmtBF16><<<grid_kv, 512, 0, s>>>(a);
      attn_bwd_dq_tile_kernel<64, FmtBF16><<<grid_q, 256, 0, s>>>(a);
    }
    return lz_check_launch("lz_attn_bwd");
  }
  if (mfma && dtype == LZ_BF16) {
    LZ_REQUIRE(qt && kt && dot, "lz_attn_bwd: MFMA path needs the transposed Q, K and dO buffers");
    AttnArgs a{};
    a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
    a.ldq = ldq; a.ldk = ldk; a.ldv = ldv;
    a.lse = const_cast<float*>(lse);
    a.qt = (const uint16_t*)qt; a.kt = (const uint16_t*)kt; a.dout = (const uint16_t*)dout; a.lddo = lddo;
    a.dot = (const uint16_t*)dot; a.delta = delta;
    a.dq = (uint16_t*)dq; a.dk = (uint16_t*)dk; a.dv = (uint16_t*)dv;
    a.lddq = lddq; a.lddk = lddk; a.lddv = lddv;
    a.rcos = (const uint16_t*)rope_cos; a.rsin = (const uint16_t*)rope_sin;
    rope_done = true;
    a.B = (int)B; a.S = (int)S; a.H = (int)H; a.KV = (int)KV; a.scale = scale;
    const unsigned grid_kv = (unsigned)(lz_cdiv(S, 128) * B * KV);
    const unsigned grid_q = (unsigned)(lz_cdiv(S, 128) * B * H);
    if (hd == 128) {
      attn_bwd_dkdv_kernel<128><<<grid_kv, 256, 0, s>>>(a);
      attn_bwd_dq_kernel<128><<<grid_q, 256, 0, s>>>(a);
    } else {
      attn_bwd_dkdv_kernel<64><<<grid_kv, 256, 0, s>>>(a);
      attn_bwd_dq_kernel<64><<<grid_q, 256, 0, s>>>(a);
    }
    return lz_check_launch("lz_attn_bwd");
  }
  const unsigned grid_q = (unsigned)lz_cdiv(B * H * S, 4);
  const unsigned grid_kv = (unsigned)lz_cdiv(B * KV * S, 4);
  if (dtype == LZ_BF16) {
    GenArgs<uint16_t> a{};
    a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
    a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.lse = const_cast<float*>(lse);
    a.dout = (const uint16_t*)dout; a.lddo = lddo; a.delta = delta;
    a.dq = (uint16_t*)dq; a.dk = (uint16_t*)dk; a.dv = (uint16_t*)dv; a.lddq = lddq; a.lddk = lddk; a.lddv = lddv;
    a.B = (int)B; a.S = (int)S; a.H = (int)H; a.KV = (int)KV; a.hd = (int)hd; a.scale = scale;
    if (hd == 16 || hd == 32) {
      launch_bwd_small(a, s);
    } else {
      attn_bwd_dq_generic_kernel<uint16_t><<<grid_q, 256, 0, s>>>(a);
      attn_bwd_dkdv_generic_kernel<uint16_t><<<grid_kv, 256, 0, s>>>(a);
    }
  } else if (dtype == LZ_F16) {
    GenArgs<_Float16> a{};
    a.q = (const _Float16*)q; a.k = (const _Float16*)k; a.v = (const _Float16*)v;
    a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.lse = const_cast<float*>(lse);
    a.dout = (const _Float16*)dout; a.lddo = lddo; a.delta = delta;
    a.dq = (_Float16*)dq; a.dk = (_Float16*)dk; a.dv = (_Float16*)dv; a.lddq = lddq; a.lddk = lddk; a.lddv = lddv;
    a.B = (int)B; a.S = (int)S; a.H = (int)H; a.KV = (int)KV; a.hd = (int)hd; a.scale = scale;
    if (hd == 16 || hd == 32) {
      launch_bwd_small(a, s);
    } else {
      attn_bwd_dq_generic_kernel<_Float16><<<grid_q, 256, 0, s>>>(a);
      attn_bwd_dkdv_generic_kernel<_Float16><<<grid_kv, 256, 0, s>>>(a);
    }
  } else if (dtype == LZ_F32) {
    GenArgs<float> a{};
    a.q = (const float*)q; a.k = (const float*)k; a.v = (const float*)v;
    a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.lse = const_cast<float*>(lse);
    a.dout = (const float*)dout; a.lddo = lddo; a.delta = delta;
    a.dq = (float*)dq; a.dk = (float*)dk; a.dv = (float*)dv; a.lddq = lddq; a.lddk = lddk; a.lddv = lddv;
    a.B = (int)B; a.S = (int)S; a.H = (int)H; a.KV = (int)KV; a.hd = (int)hd; a.scale = scale;
    if (hd == 16 || hd == 32) {
      launch_bwd_small(a, s);
    } else {
      attn_bwd_dq_generic_kernel<float><<<grid_q, 256, 0, s>>>(a);
      attn_bwd_dkdv_generic_kernel<float><<<grid_kv, 256, 0, s>>>(a);
    }
  } else {
    return lz_set_error(LZ_EINVAL, "lz_attn_bwd: bad dtype %d", dtype);
  }
  return lz_check_launch("lz_attn_bwd(generic)");
}

}  // namespace

namespace {

template <typename T>
int general_args(GenArgs<T>& a, const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                 const void* mask, int mask_kind, const int64_t* mstride, float dropout_p, uint64_t seed, int64_t B,
                 int64_t S, int64_t H, int64_t KV, int64_t hd, float scale) {
  a.q = (const T*)q; a.k = (const T*)k; a.v = (const T*)v;
  a.ldq = ldq; a.ldk = ldk; a.ldv = ldv;
  a.B = (int)B; a.S = (int)S; a.H = (int)H; a.KV = (int)KV; a.hd = (int)hd; a.scale = scale;
  a.mask = mask; a.mask_kind = mask_kind;
  if (mask_kind) {
    a.msb = mstride[0]; a.msh = mstride[1]; a.msq = mstride[2]; a.msk = mstride[3];
  }
  a.drop_thresh = (uint32_t)std::min(std::ceil((double)dropout_p * 16777216.0), 16777216.0);
  a.drop_scale = dropout_p < 1.f ? 1.0f / (1.0f - dropout_p) : 0.f;
  a.drop_seed = seed;
  return LZ_OK;
}

int check_general(const void* mask, int mask_kind, const int64_t* mstride, float dropout_p) {
  LZ_REQUIRE(mask_kind >= 0 && mask_kind <= 4, "attention mask: kind %d (0 causal, 1 bool, 2 fp32, 3 bf16, 4 fp16)",
             mask_kind);
  if (mask_kind) {
    LZ_REQUIRE(mask && mstride, "attention mask: null pointer");
    for (int i = 0; i < 4; ++i) LZ_REQUIRE(mstride[i] >= 0, "attention mask: negative stride");
  }
  LZ_REQUIRE(dropout_p >= 0.f && dropout_p <= 1.f, "attention dropout p %g not in [0, 1]", (double)dropout_p);
  return LZ_OK;
}

}  // namespace

// Attention on the one-wave-per-row kernels with the options the tile paths
// do not take (model/llama.py:109-117, F.scaled_dot_product_attention):
//   - an explicit mask in place of the causal one (attn_mask with
//     is_causal=False): mask_kind 1 = bool bytes (nonzero: the key takes
//     part), 2 = fp32, 3 = bf16, 4 = fp16 (added to the scaled scores); mstride = its
//     element strides over [B, H, S(query), S(key)], 0 where it broadcasts;
//     mask_kind 0 = causal (mask and mstride ignored).  A row whose keys are
//     all masked gives NaN, as the reference's softmax of an all -inf row does;
//   - attention dropout (dropout_p): each probability kept with scale
//     1/(1-p) by element ((b*H + h)*S + s)*S + kv of seed's stream (the
//     stream lz_dropout uses), the normaliser summing them before dropout.
// Any head dim up to 256, bf16 or fp32.
LZ_EXPORT int lz_attn_fwd_general(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                                  const void* mask, int mask_kind, const int64_t* mstride, float dropout_p,
                                  uint64_t seed, void* o, int64_t ldo, float* lse, int64_t B, int64_t S, int64_t H,
                                  int64_t KV, int64_t hd, float scale, int dtype, void* stream) {
  int rc = check_shape(B, S, H, KV, hd);
  if (rc) return rc;
  rc = check_general(mask, mask_kind, mstride, dropout_p);
  if (rc) return rc;
  LZ_REQUIRE(q && k && v && o && lse, "lz_attn_fwd_general: null pointer");
  hipStream_t s = lz_stream(stream);
  const unsigned grid = (unsigned)lz_cdiv(B * H * S, 4);
  if (dtype == LZ_BF16) {
    GenArgs<uint16_t> a{};
    general_args(a, q, ldq, k, ldk, v, ldv, mask, mask_kind, mstride, dropout_p, seed, B, S, H, KV, hd, scale);
    a.o = (uint16_t*)o; a.ldo = ldo; a.lse = lse;
    attn_fwd_generic_kernel<uint16_t><<<grid, 256, 0, s>>>(a);
  } else if (dtype == LZ_F16) {
    GenArgs<_Float16> a{};
    general_args(a, q, ldq, k, ldk, v, ldv, mask, mask_kind, mstride, dropout_p, seed, B, S, H, KV, hd, scale);
    a.o = (_Float16*)o; a.ldo = ldo; a.lse = lse;
    attn_fwd_generic_kernel<_Float16><<<grid, 256, 0, s>>>(a);
  } else if (dtype == LZ_F32) {
    GenArgs<float> a{};
    general_args(a, q, ldq, k, ldk, v, ldv, mask, mask_kind, mstride, dropout_p, seed, B, S, H, KV, hd, scale);
    a.o = (float*)o; a.ldo = ldo; a.lse = lse;
    attn_fwd_generic_kernel<float><<<grid, 256, 0, s>>>(a);
  } else {
    return lz_set_error(LZ_EINVAL, "lz_attn_fwd_general: bad dtype %d", dtype);
  }
  return lz_check_launch("lz_attn_fwd_general");
}

// Backward of lz_attn_fwd_general (same mask, dropout p and seed); delta
// from lz_attn_delta.
LZ_EXPORT int lz_attn_bwd_general(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
                                  const void* dout, int64_t lddo, const float* lse, const float* delta,
                                  const void* mask, int mask_kind, const int64_t* mstride, float dropout_p,
                                  uint64_t seed, void* dq, int64_t lddq, void* dk, int64_t lddk, void* dv,
                                  int64_t lddv, int64_t B, int64_t S, int64_t H, int64_t KV, int64_t hd, float scale,
                                  int dtype, void* stream) {
  int rc = check_shape(B, S, H, KV, hd);
  if (rc) return rc;
  rc = check_general(mask, mask_kind, mstride, dropout_p);
  if (rc) return rc;
  LZ_REQUIRE(q && k && v && dout && lse && delta && dq && dk && dv, "lz_attn_bwd_general: null pointer");
  hipStream_t s = lz_stream(stream);
  const unsigned grid_q = (unsigned)lz_cdiv(B * H * S, 4);
  const unsigned grid_kv = (unsigned)lz_cdiv(B * KV * S, 4);
  if (dtype == LZ_BF16) {
    GenArgs<uint16_t> a{};
    general_args(a, q, ldq, k, ldk, v, ldv, mask, mask_kind, mstride, dropout_p, seed, B, S, H, KV, hd, scale);
    a.lse = const_cast<float*>(lse); a.dout = (const uint16_t*)dout; a.lddo = lddo; a.delta = delta;
    a.dq = (uint16_t*)dq; a.dk = (uint16_t*)dk; a.dv = (uint16_t*)dv; a.lddq = lddq; a.lddk = lddk; a.lddv = lddv;
    attn_bwd_dq_generic_kernel<uint16_t><<<grid_q, 256, 0, s>>>(a);
    attn_bwd_dkdv_generic_kernel<uint16_t><<<grid_kv, 256, 0, s>>>(a);
  } else if (dtype == LZ_F16) {
    GenArgs<_Float16> a{};
    general_args(a, q, ldq, k, ldk, v, ldv, mask, mask_kind, mstride, dropout_p, seed, B, S, H, KV, hd, scale);
    a.lse = const_cast<float*>(lse); a.dout = (const _Float16*)dout; a.lddo = lddo; a.delta = delta;
    a.dq = (_Float16*)dq; a.dk = (_Float16*)dk; a.dv = (_Float16*)dv; a.lddq = lddq; a.lddk = lddk; a.lddv = lddv;
    attn_bwd_dq_generic_kernel<_Float16><<<grid_q, 256, 0, s>>>(a);
    attn_bwd_dkdv_generic_kernel<_Float16><<<grid_kv, 256, 0, s>>>(a);
  } else if (dtype == LZ_F32) {
    GenArgs<float> a{};
    general_args(a, q, ldq, k, ldk, v, ldv, mask, mask_kind, mstride, dropout_p, seed, B, S, H, KV, hd, scale);
    a.lse = const_cast<float*>(lse); a.dout = (const float*)dout; a.lddo = lddo; a.delta = delta;
    a.dq = (float*)dq; a.dk = (float*)dk; a.dv = (float*)dv; a.lddq = lddq; a.lddk = lddk; a.lddv = lddv;
    attn_bwd_dq_generic_kernel<float><<<grid_q, 256, 0, s>>>(a);
    attn_bwd_dkdv_generic_kernel<float><<<grid_kv, 256, 0, s>>>(a);
  } else {
    return lz_set_error(LZ_EINVAL, "lz_attn_bwd_general: bad dtype %d", dtype);
  }
  return lz_check_launch("lz_attn_bwd_general");
}
