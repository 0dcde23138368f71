// Shared device helpers for the gfx950 (MI355X) kernels of the Qwen3 int8 decode path.
//
// Conventions used by every kernel in this directory:
//   * bf16 values travel as uint16_t bit patterns. Sums that decide a rounded output are
//     accumulated in fp64 (exact to within 2^-50 for these magnitudes), so every operator
//     boundary is the correctly rounded value; the fp32 variants (decode attention with
//     IRON_ACCUM_F32, prefill, the MFMA group sums) say so where they are defined.
//   * fp32 -> bf16 is round-to-nearest-even, the rounding the reference applies at every
//     operator boundary (iron/common/sequence.py:997-999) and inside its kernels
//     (aie_kernels/aie2p/mv_int8_signed.cc:66 sets conv_even).
//   * A wavefront is 64 lanes; reductions use DPP row/bcast controls, not LDS.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#define IRON_DEV __device__ __forceinline__

// s_waitcnt immediate: vmcnt(0), expcnt and lgkmcnt unconstrained (gfx9 encoding)
constexpr int kWaitVmcnt0 = (0x7 << 4) | (0xF << 8);
// Buffer resource word 3 for raw (stride 0) buffers on CDNA: 32-bit data format, no swizzle.
constexpr int kBufferDword3 = 0x00020000;
// Cache-policy operand of the buffer builtins: sc1 (device scope: the load misses this XCD's L2).
constexpr int kCpolSc1 = 16;

// ---------------------------------------------------------------------------------------------
// bf16 <-> fp32
// ---------------------------------------------------------------------------------------------
IRON_DEV float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }
IRON_DEV float bf16lo_to_f32(uint32_t packed) { return __uint_as_float(packed << 16); }
IRON_DEV float bf16hi_to_f32(uint32_t packed) { return __uint_as_float(packed & 0xffff0000u); }

// fp32 -> bf16 with round to nearest, ties to even: one gfx950 instruction (v_cvt_pk_bf16_f32). A
// NaN stays a NaN. iron_test_bf16_round checks it against f32_to_bf16_rne on every fp32 value.
// The empty asm pins the fp32 operand: for an fp32 value just rounded from fp64 the compiler would
// otherwise fuse the two roundings into one from fp64 (round to odd, then to even), which
// differs from rounding twice, the torch semantics every caller relies on.
IRON_DEV uint16_t f32_to_bf16(float f) {
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// The same rounding in integer arithmetic (NaN -> the quiet NaN with the input's sign and top
// payload bits): the reference form the hardware conversion is checked against.
IRON_DEV uint16_t f32_to_bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t qnan = (u >> 16) | 0x40u;
  return (uint16_t)(((u & 0x7fffffffu) > 0x7f800000u) ? qnan : rne);
}
IRON_DEV float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// An fp32 value as three bf16 planes: hi = v truncated to bf16, mid = the remainder truncated,
// lo = what is left (at most 8 significant bits, so exact). hi + mid + lo == v exactly, so a
// product of a bf16 with each plane, summed in fp32 or wider, sees the fp32 value.
IRON_DEV void split3_bf16(float v, uint16_t& hi, uint16_t& mid, uint16_t& lo) {
  const float h = __uint_as_float(__float_as_uint(v) & 0xffff0000u);
  const float r = v - h;
  const float m = __uint_as_float(__float_as_uint(r) & 0xffff0000u);
  hi = (uint16_t)(__float_as_uint(h) >> 16);
  mid = (uint16_t)(__float_as_uint(m) >> 16);
  lo = (uint16_t)(__float_as_uint(r - m) >> 16);
}

// fp64 -> bf16 goes through fp32 (RNE at each step), the conversion path torch uses for a
// float64 tensor cast to bfloat16, so device results and the fp64 oracle round identically.
IRON_DEV uint16_t f64_to_bf16(double d) { return f32_to_bf16((float)d); }

// ---------------------------------------------------------------------------------------------
// Loads and stores through the global address space. A pointer the compiler cannot trace to a
// kernel argument (one read from device memory) is generic, and generic accesses compile to FLAT
// instructions, whose completion waits the compiler can only place as vmcnt(0). These helpers make
// the access a global one, counted in order with the other vector memory operations.
// ---------------------------------------------------------------------------------------------
template <class T>
IRON_DEV T ld_global(const T* p) {
  return *(const __attribute__((address_space(1))) T*)p;
}

template <class T>
IRON_DEV void st_global(T* p, const T& v) {
  *(__attribute__((address_space(1))) T*)p = v;
}

// 16-byte accesses go through a native vector type: HIP's uint4 copies through a generic `this`.
typedef unsigned int iron_u32x4 __attribute__((ext_vector_type(4)));

template <>
IRON_DEV uint4 ld_global<uint4>(const uint4* p) {
  const iron_u32x4 v = *(const __attribute__((address_space(1))) iron_u32x4*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}

typedef unsigned int iron_u32x2 __attribute__((ext_vector_type(2)));

template <>
IRON_DEV uint2 ld_global<uint2>(const uint2* p) {
  const iron_u32x2 v = *(const __attribute__((address_space(1))) iron_u32x2*)p;
  return make_uint2(v.x, v.y);
}

template <>
IRON_DEV void st_global<uint4>(uint4* p, const uint4& v) {
  const iron_u32x4 u = {v.x, v.y, v.z, v.w};
  *(__attribute__((address_space(1))) iron_u32x4*)p = u;
}

// ---------------------------------------------------------------------------------------------
// Wavefront reductions (wave64) with DPP. The moves leave the destination of lanes they do not
// write undefined (no old value, which would cost a move per 32 bits): every control used here
// writes every lane, except the row_bcast steps of wave_sum*, whose unwritten rows (0 and 2,
// then 0 and 1) are never read again -- the total is taken from lane 63.
// ---------------------------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
IRON_DEV float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, ROW_MASK, BANK_MASK,
                                                 false));
}

// Sum over each 16-lane row; every lane of the row receives the row's sum.
IRON_DEV float row16_sum(float v) {
  v += dpp_f<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  return v;
}

// Sum over the full wavefront; every lane receives the total.
IRON_DEV float wave_sum(float v) {
  v = row16_sum(v);
  v += dpp_f<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_f<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

IRON_DEV float row16_max(float v) {
  v = fmaxf(v, dpp_f<0xb1>(v));
  v = fmaxf(v, dpp_f<0x4e>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return v;
}

IRON_DEV float wave_max(float v) {
  // every lane receives the maximum, so the cross-row steps are xor-shuffles (a row_bcast step
  // leaves rows unwritten)
  v = row16_max(v);
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

// ---- fp64 variants: DPP moves 32 bits, so a double is moved as two halves.
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
IRON_DEV double dpp_d(double v) {
  const int lo = __builtin_amdgcn_mov_dpp(__double2loint(v), CTRL, ROW_MASK, BANK_MASK, false);
  const int hi = __builtin_amdgcn_mov_dpp(__double2hiint(v), CTRL, ROW_MASK, BANK_MASK, false);
  return __hiloint2double(hi, lo);
}

IRON_DEV double row16_sum_d(double v) {
  v += dpp_d<0xb1>(v);
  v += dpp_d<0x4e>(v);
  v += dpp_d<0x141>(v);
  v += dpp_d<0x140>(v);
  return v;
}

IRON_DEV double wave_sum_d(double v) {
  v = row16_sum_d(v);
  v += dpp_d<0x142, 0xa>(v);
  v += dpp_d<0x143, 0xc>(v);
  const int lo = __builtin_amdgcn_readlane(__double2loint(v), 63);
  const int hi = __builtin_amdgcn_readlane(__double2hiint(v), 63);
  return __hiloint2double(hi, lo);
}

IRON_DEV double row16_max_d(double v) {
  v = fmax(v, dpp_d<0xb1>(v));
  v = fmax(v, dpp_d<0x4e>(v));
  v = fmax(v, dpp_d<0x141>(v));
  v = fmax(v, dpp_d<0x140>(v));
  return v;
}

// 1 / sqrt(v) in fp64 for v > 0: the hardware reciprocal square root (about 24 correct bits)
// refined by two Newton steps, y <- y + y (1 - v y^2) / 2, to within a few units of 2^-53 of the
// correctly rounded value. The bf16 / fp32 values the kernels compute from it then round exactly
// like the correctly rounded form except when they sit that close to a rounding boundary.
IRON_DEV double rsqrt_d(double v) {
  double y = __builtin_amdgcn_rsq(v);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const double e = fma(-v * y, y, 1.0);
    y = fma(0.5 * y, e, y);
  }
  return y;
}

// The RMSNorm factor 1 / sqrt(ss / n + eps); for n a power of two the mean is an exact scaling.
IRON_DEV double inv_rms(double ss, int n, double eps) {
  const double mean = (n & (n - 1)) == 0 ? ldexp(ss, -(31 - __clz(n))) : ss / (double)n;
  return rsqrt_d(mean + eps);
}

// Sum of squares of N exact fp32 values in fp64 as a balanced tree (depth log2 N; every square
// and partial sum of bf16-derived values is exact in fp64 for the magnitudes involved).
template <int N>
IRON_DEV double sum_sq_tree(const double (&v)[N]) {
  double t[N];
#pragma unroll
  for (int i = 0; i < N; ++i) t[i] = v[i] * v[i];
#pragma unroll
  for (int w = N / 2; w >= 1; w >>= 1)
#pragma unroll
    for (int i = 0; i < w; ++i) t[i] += t[i + w];
  return t[0];
}

// Block-wide fp64 sum for blockDim.x == 256. `scratch` holds >= 4 doubles of LDS.
IRON_DEV double block_sum_256_d(double v, double* scratch) {
  v = wave_sum_d(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  __syncthreads();
  return (scratch[0] + scratch[1]) + (scratch[2] + scratch[3]);
}

// Block-wide sum for blockDim.x == 256 (4 waves). `scratch` holds >= 4 floats of LDS.
IRON_DEV float block_sum_256(float v, float* scratch) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  __syncthreads();
  float t = scratch[0] + scratch[1] + scratch[2] + scratch[3];
  return t;
}

// ---------------------------------------------------------------------------------------------
// Division by a runtime constant (rows -> wire blocks), valid for 0 <= n < 2^31.
//   l = ceil(log2 d), m = floor(2^32 * (2^l - d) / d) + 1, q = (umulhi(m, n) + n) >> l
// ---------------------------------------------------------------------------------------------
struct FastDiv {
  uint32_t m;
  uint32_t l;
  uint32_t d;
};

static inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  f.l = l;
  f.m = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1ull);
  f.d = d;
  return f;
}

IRON_DEV uint32_t fastdiv(uint32_t n, FastDiv f) {
  uint32_t t = __umulhi(f.m, n);
  return (t + n) >> f.l;
}

static inline uint32_t fastdiv_host(uint32_t n, FastDiv f) {
  uint32_t t = (uint32_t)(((uint64_t)f.m * n) >> 32);
  return (t + n) >> f.l;
}

// ---------------------------------------------------------------------------------------------
// Cross-workgroup hand-off: the "last workgroup to finish does the merge" pattern. Writers make
// their results visible device-wide (agent-scope release), then count in; the workgroup that
// completes the count acquires and merges, then resets the counter so the next launch (or graph
// replay) starts from zero without a memset.
// ---------------------------------------------------------------------------------------------
IRON_DEV bool arrive_is_last(unsigned int* counter, unsigned int expected) {
  __shared__ unsigned int s_last;
  __syncthreads();
  if (threadIdx.x == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    unsigned int prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == expected - 1u) ? 1u : 0u;
    if (s_last) {
      __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
  }
  __syncthreads();
  return s_last != 0u;
}

// The same hand-off without the agent-scope fences, for results the writers store write-through
// (st_agent: agent-scope stores complete at the device's coherence point, past this XCD's L2) and
// the merger reads with ld_agent_* (sc1 loads miss this XCD's L2, so no line it cached from an
// earlier launch is seen). Each thread waits for its own stores (vmcnt 0) before the barrier, so
// the count follows every store of the workgroup. An agent-scope release fence would instead
// write back this XCD's whole L2 (buffer_wbl2) in every arriving workgroup, and the acquire would
// invalidate it.
IRON_DEV bool arrive_is_last_wt(unsigned int* counter, unsigned int expected) {
  __shared__ unsigned int s_last_wt;
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned int prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
    s_last_wt = (prev == expected - 1u) ? 1u : 0u;
    if (s_last_wt) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return s_last_wt != 0u;
}

IRON_DEV void st_agent(double* p, double v) {
  __hip_atomic_store((unsigned long long*)p, (unsigned long long)__double_as_longlong(v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
IRON_DEV void st_agent(float* p, float v) {
  __hip_atomic_store((unsigned int*)p, __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// sc1 loads of 8 or 16 bytes at byte offset `off` of a raw buffer (up to 2 GiB).
IRON_DEV __amdgpu_buffer_rsrc_t agent_rsrc(const void* base, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kBufferDword3);
}
IRON_DEV iron_u32x2 ld_agent_b64(__amdgpu_buffer_rsrc_t rs, int off) {
  return __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, kCpolSc1);
}
IRON_DEV iron_u32x4 ld_agent_b128(__amdgpu_buffer_rsrc_t rs, int off) {
  return __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kCpolSc1);
}
