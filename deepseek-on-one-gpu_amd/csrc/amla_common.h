// Shared device helpers for the gfx950 (CDNA4) MLA + block-FP8 kernels.
//
// Conventions
//  * bf16 values travel as uint16_t bit patterns; conversions are exact
//    (bf16 -> f32 is a shift) or round-to-nearest-even (f32 -> bf16, the same
//    rounding torch uses for .to(torch.bfloat16)).
//  * fp8 is OCP e4m3fn (the gfx950 native format, identical to
//    torch.float8_e4m3fn): the hardware convert to f32 is exact.
//  * MFMA tile v_mfma_f32_16x16x32_bf16 (wave64):
//      A (16 x 32): lane l holds row l%16, k = 8*(l/16) .. +7
//      B (32 x 16): lane l holds col l%16, k = 8*(l/16) .. +7
//      C (16 x 16): lane l holds col l%16, rows 4*(l/16) .. +3
//    Any permutation of k that A and B share gives the same product, which the
//    kernels use to load contiguous bytes per lane.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define AMLA_DEV __device__ __forceinline__

namespace amla {

AMLA_DEV float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

AMLA_DEV uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Round an f32 through bf16 and back (the value a bf16 tensor would hold).
AMLA_DEV float round_bf16(float f) { return bf2f(f2bf(f)); }

// Low / high bf16 of a packed dword, as f32.
AMLA_DEV float lo_bf(uint32_t v) { return __uint_as_float(v << 16); }
AMLA_DEV float hi_bf(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

AMLA_DEV uint32_t pack_bf16(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));  // v_cvt_pk_bf16_f32, RNE
}

// Two e4m3fn bytes (bytes 0,1 or 2,3 of w) -> two exact f32.
template <bool HI>
AMLA_DEV f32x2 fp8x2_to_f32(uint32_t w) {
  return __builtin_amdgcn_cvt_pk_f32_fp8((int)w, HI);
}

// Four e4m3fn bytes -> four bf16 packed in two dwords.  Exact: every e4m3
// value has <= 4 significant bits and an exponent bf16 covers, so taking the
// high half of the exact f32 loses nothing.
AMLA_DEV u32x2 fp8x4_to_bf16x4(uint32_t w) {
  f32x2 a = fp8x2_to_f32<false>(w);
  f32x2 b = fp8x2_to_f32<true>(w);
  u32x2 r;
  r.x = __builtin_amdgcn_perm(__float_as_uint(a.y), __float_as_uint(a.x), 0x07060302u);
  r.y = __builtin_amdgcn_perm(__float_as_uint(b.y), __float_as_uint(b.x), 0x07060302u);
  return r;
}

// 16 e4m3fn bytes -> two MFMA operands of 8 bf16 each.
AMLA_DEV void fp8x16_to_bf16x16(u32x4 w, bf16x8 &lo, bf16x8 &hi) {
  u32x2 p0 = fp8x4_to_bf16x4(w.x), p1 = fp8x4_to_bf16x4(w.y);
  u32x2 p2 = fp8x4_to_bf16x4(w.z), p3 = fp8x4_to_bf16x4(w.w);
  u32x4 a = {p0.x, p0.y, p1.x, p1.y};
  u32x4 b = {p2.x, p2.y, p3.x, p3.y};
  lo = __builtin_bit_cast(bf16x8, a);
  hi = __builtin_bit_cast(bf16x8, b);
}

AMLA_DEV f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

AMLA_DEV u32x4 ldg16(const void *p) { return *reinterpret_cast<const u32x4 *>(p); }
AMLA_DEV u32x2 ldg8(const void *p) { return *reinterpret_cast<const u32x2 *>(p); }

AMLA_DEV u32x4 ldg16_nt(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}
AMLA_DEV u32x2 ldg8_nt(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p));
}

AMLA_DEV bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// LDS address operand of __builtin_amdgcn_global_load_lds
#define LDS_PTR(p) ((__attribute__((address_space(3))) void *)(p))

// Wait until at most N of this wave's vector memory operations are in flight
// (global_load_lds copies included).
template <int N>
AMLA_DEV void wait_vmcnt() {
  if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory");
}

// Butterfly reductions inside a wave.
AMLA_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

AMLA_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace amla
