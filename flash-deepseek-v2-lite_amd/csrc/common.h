// Shared device helpers for the gfx950 (CDNA4) decode-step kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dsv2lite.h"

typedef uint16_t bf16_t;  // raw bf16 bits; all arithmetic is done in fp32
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

#define DSV2_WAVE 64

// ---- host-side error plumbing ----------------------------------------------
void dsv2_set_error(const char* fmt, ...);
int dsv2_launch_status(const char* what);

#define DSV2_REQUIRE(cond, code, ...)  \
  do {                                 \
    if (!(cond)) {                     \
      dsv2_set_error(__VA_ARGS__);     \
      return (code);                   \
    }                                  \
  } while (0)

static inline bool dsv2_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- bf16 <-> fp32 ---------------------------------------------------------
__device__ __forceinline__ float bf2f(bf16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// round-to-nearest-even, NaN kept quiet (torch's float->bfloat16 conversion)
__device__ __forceinline__ bf16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<bf16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<bf16_t>(u >> 16);
}

// value of f after rounding to bf16, as fp32
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
  f[0] = __uint_as_float(v.x << 16);
  f[1] = __uint_as_float(v.x & 0xffff0000u);
  f[2] = __uint_as_float(v.y << 16);
  f[3] = __uint_as_float(v.y & 0xffff0000u);
  f[4] = __uint_as_float(v.z << 16);
  f[5] = __uint_as_float(v.z & 0xffff0000u);
  f[6] = __uint_as_float(v.w << 16);
  f[7] = __uint_as_float(v.w & 0xffff0000u);
}

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return static_cast<uint32_t>(f2bf(lo)) | (static_cast<uint32_t>(f2bf(hi)) << 16);
}

__device__ __forceinline__ uint4 pack8(const float* f) {
  uint4 v;
  v.x = pack2(f[0], f[1]);
  v.y = pack2(f[2], f[3]);
  v.z = pack2(f[4], f[5]);
  v.w = pack2(f[6], f[7]);
  return v;
}

__device__ __forceinline__ uint4 ldg16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// 16-byte load with the non-temporal hint, for the weight streams of the few-row GEMVs:
// on MI355X a 256-CU stream of such loads reaches ~6.8 TB/s from HBM against ~6.1 TB/s for
// plain loads, but one CU then streams ~62 GB/s instead of ~130 GB/s -- so kernels whose
// bytes sit on few CUs, and the MFMA GEMMs (measured slower), keep plain loads.  The hint
// only changes the cache policy, not coherence.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16 (gfx950): in each 16-lane group, lane i receives element i % 4 of the
// four 16-bit elements that lane 4e + i / 4 addressed, for e = 0..3 (measured with a probe
// kernel on MI355X: LDS element values = their index).  p must point into LDS, 8-byte aligned.
// s_waitcnt immediate (gfx9 encoding): wait until at most n vector-memory operations are
// outstanding, leaving the LDS/scalar (15) and export (7) counters unconstrained
constexpr int vmcnt_only(int n) { return (n & 0xf) | (0x7 << 4) | (0xf << 8) | (((n >> 4) & 3) << 14); }
__device__ __forceinline__ uint2 lds_read_tr16(const bf16_t* p) {
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  const bf16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4_t*)p);
  return __builtin_bit_cast(uint2, v);
}
__device__ __forceinline__ uint4 ldg16_nt(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// v if ok else 0, component-wise (a `?:` between two uint4 values is lowered through
// scratch memory; a mask keeps it in registers)
__device__ __forceinline__ uint4 keep_if(bool ok, const uint4& v) {
  const uint32_t m = ok ? 0xffffffffu : 0u;
  return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
}

// Holds a loaded value at this point of the program.  Loads complete in issue order, and
// the compiler moves a load that is used only inside a branch into that branch (or turns a
// select between two loads into one); the wait for it there also waits for every load
// issued before it -- typically a weight stream.  Pinning an early operand (x, norm weights,
// residuals) right after the weight loads are issued keeps its load ahead of them, and the
// wait here covers only the loads issued before it.
__device__ __forceinline__ void pin(uint32_t v) { asm volatile("" ::"v"(v)); }

// 16 fp8 (OCP e4m3, the format of gfx950's v_cvt_pk_f32_fp8) -> fp32, two per instruction
__device__ __forceinline__ void unpack16_fp8(const uint4& v, float* f) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[i]), false);
    const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[i]), true);
    f[4 * i] = lo[0];
    f[4 * i + 1] = lo[1];
    f[4 * i + 2] = hi[0];
    f[4 * i + 3] = hi[1];
  }
}

__device__ __forceinline__ float dot16_fp8(const uint4& w, const float* x) {
  float f[16];
  unpack16_fp8(w, f);
  float s = f[0] * x[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) s = __builtin_fmaf(f[i], x[i], s);
  return s;
}

__device__ __forceinline__ float dot8(const uint4& w, const float* x) {
  float f[8];
  unpack8(w, f);
  float s = f[0] * x[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) s = __builtin_fmaf(f[i], x[i], s);
  return s;
}

// ---- wave / block reductions (wave64) ---------------------------------------
// v combined with lane l ^ 32 (xor32_*) or l ^ 16 (xor16_*) by the gfx950 VALU lane swaps
// instead of LDS-routed shuffles: v_permlane32_swap on two copies of v leaves [lo, lo] in
// one and [hi, hi] in the other (the wave's 32-lane halves), v_permlane16_swap does the same
// for rows 0 / 1 and 2 / 3; op(a, b) is symmetric, so every lane gets exactly the value of
// v op __shfl_xor(v, 32 or 16) (checked bit for bit on MI355X)
__device__ __forceinline__ float xor32_sum(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float xor16_sum(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

#define DSV2_DPP(v, ctrl) \
  __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, (v)), (ctrl), 0xF, 0xF, false))
// v at lane l ^ off for off = 1, 2, 4, 8 by DPP within the 16-lane rows: quad_perm [1,0,3,2]
// and [2,3,0,1], row_ror:8, and for 4 row_shl:4 / row_shr:4 chosen by lane bit 2 (each the
// exact xor partner, checked against __shfl_xor on MI355X)
__device__ __forceinline__ float xor_partner_row(float v, int off) {
  if (off == 1) return DSV2_DPP(v, 0xB1);
  if (off == 2) return DSV2_DPP(v, 0x4E);
  if (off == 8) return DSV2_DPP(v, 0x128);
  const float up = DSV2_DPP(v, 0x104), dn = DSV2_DPP(v, 0x114);
  return (threadIdx.x & 4) ? dn : up;
}
// one butterfly step, v op (v at lane l ^ off), off a compile-time constant in the unrolled
// loops that call these: lane swaps for 32 and 16, DPP below -- no LDS-routed shuffles
__device__ __forceinline__ float xor_sum(float v, int off) {
  return off == 32 ? xor32_sum(v) : (off == 16 ? xor16_sum(v) : v + xor_partner_row(v, off));
}
__device__ __forceinline__ float xor_max(float v, int off) {
  return off == 32 ? xor32_max(v) : (off == 16 ? xor16_max(v) : fmaxf(v, xor_partner_row(v, off)));
}

// butterfly over the 64 lanes, l ^ 32 first (every lane gets the same, fixed-order sum)
__device__ __forceinline__ float wave_sum(float v) {
  v = xor16_sum(xor32_sum(v));
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) v = xor_sum(v, o);
  return v;
}

// Wave64 sum on the VALU: DPP within each 16-lane row (quad_perm xor 1, xor 2, then
// row_half_mirror and row_mirror leave the row's sum in all 16 lanes), then the four row
// sums read into scalars.  Uniform result; a different (fixed) summation order from
// wave_sum, with no LDS traffic and a short dependency chain.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += DSV2_DPP(v, 0xB1);   // quad_perm [1,0,3,2]
  v += DSV2_DPP(v, 0x4E);   // quad_perm [2,3,0,1]
  v += DSV2_DPP(v, 0x141);  // row_half_mirror
  v += DSV2_DPP(v, 0x140);  // row_mirror
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_max(float v) {
  v = xor16_max(xor32_max(v));
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) v = xor_max(v, o);
  return v;
}

// (value, index) max with ties resolved to the lower index
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float v2 = __shfl_xor(v, o, DSV2_WAVE);
    int i2 = __shfl_xor(i, o, DSV2_WAVE);
    if (v2 > v || (v2 == v && i2 < i)) {
      v = v2;
      i = i2;
    }
  }
}

// sum over a block of NW waves; `red` must hold NW floats of LDS
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) t += red[i];
  __syncthreads();
  return t;
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }

// HF rounding of the SwiGLU product: bf16(bf16(silu(bf16 g)) * bf16 u)
__device__ __forceinline__ float swiglu_bf(float g, float u) {
  const float gb = rbf(g);
  return rbf(rbf(silu_f(gb)) * rbf(u));
}

__device__ __forceinline__ floatx4_t mfma16x16x32(const bf16x8_t& a, const bf16x8_t& b, const floatx4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& v) { return __builtin_bit_cast(bf16x8_t, v); }
