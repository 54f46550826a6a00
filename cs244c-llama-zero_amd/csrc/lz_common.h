// Shared definitions for the llama-zero gfx950 kernels.
//
// Every exported entry point is `extern "C"`, takes raw device pointers,
// int64 sizes and a hipStream_t passed as `void*`, launches asynchronously on
// that stream and returns 0 on success or a negative status.  The message of
// the last failure on the calling thread is available from lz_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#define LZ_OK 0
#define LZ_EINVAL -1
#define LZ_ELAUNCH -2
#define LZ_ERUNTIME -3

// dtype codes shared with the Python side.
#define LZ_F32 0
#define LZ_BF16 1
#define LZ_F16 2

// Bytes per element of a dtype code.
static inline int lz_esize(int dtype) { return dtype == LZ_F32 ? 4 : 2; }

#define LZ_EXPORT extern "C" __attribute__((visibility("default")))

// Records `msg` as the last error of this thread and returns `code`.
int lz_set_error(int code, const char* fmt, ...);
// Converts a pending launch error into a status.
int lz_check_launch(const char* what);

#define LZ_REQUIRE(cond, ...)                          \
  do {                                                 \
    if (!(cond)) return lz_set_error(LZ_EINVAL, __VA_ARGS__); \
  } while (0)

static inline hipStream_t lz_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

static inline bool lz_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

__host__ __device__ static inline int64_t lz_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// bfloat16 <-> float.  Storage is uint16_t; conversion is round-to-nearest-even
// with NaN preserved, which is what torch's `.to(torch.bfloat16)` does.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats -> two bf16 packed low/high with one v_cvt_pk_bf16_f32: round to
// nearest even, NaN kept quiet with its sign.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

__device__ __forceinline__ uint16_t f2bf(float f) { return (uint16_t)(pack_bf16x2(f, 0.0f) & 0xffffu); }

// s_waitcnt with only the vector-memory counter limited to N (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Raw buffer resource (4 SGPRs) starting at `base`: stride 0, 2^31 - 1
// bytes addressable, the same flag word as __builtin_amdgcn_make_buffer_rsrc
// takes.  `base` must be wave-uniform; the words are read from the first
// active lane so that they live in SGPRs whatever the compiler can prove.
typedef int lz_v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ lz_v4i lz_buffer_rsrc(const void* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  lz_v4i r;
  r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r.y = __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
  r.z = 0x7fffffff;
  r.w = 0x00020000;
  return r;
}

// Direct-to-LDS copy, 16 bytes per lane: buffer_load_dwordx4 ... lds puts
// the 16 bytes of lane l, at byte offset voff + soff of `rsrc`, at LDS address
// dst + 16*l (dst wave-uniform; M0 carries it).  Issued from inline assembly
// so that the compiler does not track these loads: with the intrinsic it
// makes every later transposed LDS read (ds_read_b64_tr_b16) wait for all of
// them, so a stage prefetched for the next step stalls the current one.
// Nothing else waits for them either: every reader of the destination must
// pass a dma_barrier() (vmcnt(0), then the workgroup barrier) after the copy
// is issued.
__device__ __forceinline__ void lz_dma16(lz_v4i rsrc, uint32_t voff, uint32_t soff, void* dst) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)dst;
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :: "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(m0) : "memory");
}

// lz_dma16 for the first load after `rsrc` was formed: its SGPRs may have
// just been written by v_readfirstlane, and a VALU write of an SGPR must be
// followed by 5 wait states before a vector-memory instruction reads it (the
// compiler pads for its own instructions, not for inline assembly).
__device__ __forceinline__ void lz_dma16_first(lz_v4i rsrc, uint32_t voff, uint32_t soff, void* dst) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)dst;
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :: "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(m0) : "memory");
}

// 16-byte store with the nontemporal hint (global_store_dwordx4 ... nt): for
// outputs a kernel writes once and does not read back, so that they do not
// displace the operand rows the rest of the grid is still reading from L2.
typedef unsigned int lz_u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void st_nt16(void* p, const uint4& v) {
  __builtin_nontemporal_store(__builtin_bit_cast(lz_u32x4_t, v), reinterpret_cast<lz_u32x4_t*>(p));
}

// Workgroup barrier that publishes LDS written by this workgroup's
// global_load_lds (direct-to-LDS) loads: each wave first waits until its own
// loads have landed (vmcnt(0)), then the barrier orders every wave's reads
// after every wave's loads.  __syncthreads() alone does not wait for these
// loads: its fence covers stores and LDS instructions only, and the compiler
// does not always add the wait.
__device__ __forceinline__ void dma_barrier() {
  wait_vmcnt<0>();  // the builtin, so the compiler's own count of pending loads restarts from zero too
  __syncthreads();
}

// Dropout's counter-based random stream: element i of a stream with seed s
// is the i-th output of SplitMix64 (Steele, Lea and Flood, "Fast Splittable
// Pseudorandom Number Generators", OOPSLA 2014) started at s, i.e. its
// finalizer applied to s + (i + 1) * gamma.  The top 24 bits are a uniform
// draw u in [0, 2^24); the element is kept when u >= thresh, thresh =
// ceil(p * 2^24).  Any element's draw is computed on its own, so forward and
// backward regenerate the same mask from (seed, index) without storing it.
__device__ __forceinline__ uint64_t lz_splitmix64(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ bool lz_keep(uint64_t seed, uint64_t i, uint32_t thresh) {
  return (uint32_t)(lz_splitmix64(seed, i) >> 40) >= thresh;
}

// Rounds a float to the nearest bfloat16 value, kept as float.
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

// IEEE binary16 <-> float (v_cvt_f32_f16 / v_cvt_f16_f32: round to nearest
// even, overflow to infinity, as torch's `.to(torch.float16)`).  Storage is
// the 16 bits, as for bfloat16.
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) { return (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16); }
__device__ __forceinline__ float round_h(float f) { return (float)(_Float16)f; }

// The two 16-bit float formats as policies over uint16_t storage, for kernels
// written once for both: to_f / from_f / pack2 (two values, low first) /
// round (to the format and back).
struct FmtBF16 {
  static constexpr int kDtype = LZ_BF16;
  static __device__ __forceinline__ float to_f(uint32_t h) { return bf2f((uint16_t)h); }
  static __device__ __forceinline__ uint16_t from_f(float f) { return f2bf(f); }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
  static __device__ __forceinline__ float round(float f) { return round_bf(f); }
};
struct FmtF16 {
  static constexpr int kDtype = LZ_F16;
  static __device__ __forceinline__ float to_f(uint32_t h) { return h2f((uint16_t)h); }
  static __device__ __forceinline__ uint16_t from_f(float f) { return f2h(f); }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack_f16x2(lo, hi); }
  static __device__ __forceinline__ float round(float f) { return round_h(f); }
};

// sigmoid(g) = 1 / (1 + 2^(-g log2 e)) with the hardware exp2 and reciprocal
// (about 1 ulp in fp32, below the bf16 rounding of every output).
__device__ __forceinline__ float sigmoid_hw(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * g));
}

// SwiGLU forward on 8 bf16 pairs (16 bytes of gate, 16 of up): rounds
// silu(g) to bf16 before multiplying by u, as the reference's bf16 ops do
// (F.silu then the product), and rounds the product.
__device__ __forceinline__ uint4 swiglu_fwd8(const uint4& gv, const uint4& uv) {
  const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
  const uint32_t uw[4] = {uv.x, uv.y, uv.z, uv.w};
  uint32_t ow[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float g0 = bf2f(gw[k] & 0xffff), g1 = bf2f(gw[k] >> 16);
    const float u0 = bf2f(uw[k] & 0xffff), u1 = bf2f(uw[k] >> 16);
    const float h0 = round_bf(g0 * sigmoid_hw(g0)) * u0, h1 = round_bf(g1 * sigmoid_hw(g1)) * u1;
    ow[k] = pack_bf16x2(h0, h1);
  }
  return make_uint4(ow[0], ow[1], ow[2], ow[3]);
}

// SwiGLU backward on 8 bf16 triples (16 bytes each of gate, up and dh) with
// the reference's bf16 roundings (autograd of F.silu(g) * u in bf16):
//   ds = r(dh * u),  du = r(dh * r(silu(g))),
//   dg = r(ds * sigmoid(g) * (1 + g * (1 - sigmoid(g)))).
__device__ __forceinline__ void swiglu_bwd8(const uint4& gv, const uint4& uv, const uint4& hv, uint4& dgv, uint4& duv) {
  const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
  const uint32_t uw[4] = {uv.x, uv.y, uv.z, uv.w};
  const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
  uint32_t ga[4], ua[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float dg[2], du[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float gx = bf2f((uint16_t)(gw[k] >> (16 * e))), ux = bf2f((uint16_t)(uw[k] >> (16 * e)));
      const float dx = bf2f((uint16_t)(hw[k] >> (16 * e)));
      const float sig = sigmoid_hw(gx);
      const float sl = round_bf(gx * sig);
      const float ds = round_bf(dx * ux);
      du[e] = dx * sl;
      dg[e] = ds * sig * (1.0f + gx * (1.0f - sig));
    }
    ga[k] = pack_bf16x2(dg[0], dg[1]);
    ua[k] = pack_bf16x2(du[0], du[1]);
  }
  dgv = make_uint4(ga[0], ga[1], ga[2], ga[3]);
  duv = make_uint4(ua[0], ua[1], ua[2], ua[3]);
}

template <typename T>
struct Elem;

template <>
struct Elem<float> {
  static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store(float* p, int64_t i, float v) { p[i] = v; }
  // Rounding to the storage type (identity for fp32).
  static __device__ __forceinline__ float round(float v) { return v; }
};

template <>
struct Elem<uint16_t> {
  static __device__ __forceinline__ float load(const uint16_t* p, int64_t i) { return bf2f(p[i]); }
  static __device__ __forceinline__ void store(uint16_t* p, int64_t i, float v) { p[i] = f2bf(v); }
  static __device__ __forceinline__ float round(float v) { return round_bf(v); }
};

// IEEE fp16 storage.
template <>
struct Elem<_Float16> {
  static __device__ __forceinline__ float load(const _Float16* p, int64_t i) { return (float)p[i]; }
  static __device__ __forceinline__ void store(_Float16* p, int64_t i, float v) { p[i] = (_Float16)v; }
  static __device__ __forceinline__ float round(float v) { return round_h(v); }
};

// ---------------------------------------------------------------------------
// Wavefront (64-lane) and block reductions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over the whole block; every thread gets the result.  `scratch` must
// hold blockDim.x/64 floats.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  float r = 0.f;
  for (int i = 0; i < nw; ++i) r += scratch[i];
  return r;
}

__device__ __forceinline__ float block_max(float v, float* scratch) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  float r = -INFINITY;
  for (int i = 0; i < nw; ++i) r = fmaxf(r, scratch[i]);
  return r;
}

// Number of compute units of the current device (cached per device).
int lz_num_cus();
