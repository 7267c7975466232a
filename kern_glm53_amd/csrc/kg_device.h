// Device-side helpers shared by every kernel of the library (gfx950 / CDNA4, wave64).
//
// Numerics are chosen to be bit-reproducible: bf16 and e4m3 results are round-to-nearest-even (e4m3
// saturating to +-448 as CUDA's __NV_SATFINITE in the reference, source/glm_glue.cu:76-79 and
// source/glm_prep.cu:69), the UE8M0 exponent follows source/glm_glue.cu:67-74, and kg_exp is the path's
// own exp (Cody-Waite reduction, degree-7 Taylor polynomial, explicit fused multiply-adds) evaluated the
// same way on every device.  The SiLU of the MoE's gate values (always bf16) uses the hardware's exp2 and
// reciprocal instead: a function of the 65536 bf16 inputs, which the tests tabulate on the GPU.  The bf16 and packed e4m3 conversions use gfx950's conversion instructions
// (v_cvt_pk_bf16_f32, v_cvt_pk_fp8_f32); on a GPU they give the integer rounding below (kg_e4m3) bit for bit
// on every non-NaN input (bf16: all ties of every bf16 value and 4M random patterns; e4m3: every bf16 value
// times powers of two within +-448, the only inputs the path produces, as its block scales bound them).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint8_t u8;
typedef uint16_t u16;
typedef uint32_t u32;
typedef uint64_t u64;

#define KG_DEV __device__ __forceinline__

KG_DEV float kg_u2f(u32 u) { return __uint_as_float(u); }
KG_DEV u32 kg_f2u(float f) { return __float_as_uint(f); }

KG_DEV float kg_bf16_to_f32(u16 h) { return kg_u2f((u32)h << 16); }

typedef __bf16 kg_bf16x2 __attribute__((ext_vector_type(2)));

// f32 -> bf16 bits, round to nearest even (NaN -> a quiet NaN).
KG_DEV u16 kg_f32_to_bf16(float f) { return __builtin_bit_cast(u16, (__bf16)f); }

// Two f32 -> packed bf16 pair (lo in bits 0-15): one v_cvt_pk_bf16_f32.
KG_DEV u32 kg_pack_bf16x2(float lo, float hi) {
  const kg_bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(u32, v);
}

// f32 -> OCP e4m3fn, round to nearest even, saturating to +-448, NaN -> 0x7f | sign.
KG_DEV u32 kg_e4m3(float x) {
  const u32 u = kg_f2u(x);
  const u32 sign = (u >> 24) & 0x80u;
  const u32 a = u & 0x7fffffffu;
  u32 r;
  if (a > 0x7f800000u) {
    r = 0x7fu;
  } else if (a >= 0x43e00000u) {
    r = 0x7eu;
  } else if (a < 0x3c800000u) {
    r = (u32)__builtin_rintf(kg_u2f(a) * 512.0f);       // subnormal grid 2^-9, exact scaling
  } else {
    r = ((a + 0x7ffffu + ((a >> 20) & 1u)) >> 20) - ((127u - 7u) << 3);
    r = r > 0x7eu ? 0x7eu : r;
  }
  return sign | r;
}

// Four f32 within +-448 -> packed e4m3 (a in bits 0-7): two v_cvt_pk_fp8_f32, equal to kg_e4m3 on them.
KG_DEV u32 kg_e4m3x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (u32)w;
}

// OCP e4m3fn -> f32 (exact).
KG_DEV float kg_e4m3_to_f32(u32 b) {
  const u32 s = (b & 0x80u) << 24, e = (b >> 3) & 15u, m = b & 7u;
  if (e == 15u && m == 7u) return kg_u2f(s | 0x7fc00000u);
  if (e == 0u) return kg_u2f(s | kg_f2u((float)m * 0.001953125f));       // m * 2^-9
  return kg_u2f(s | ((e + 120u) << 23) | (m << 20));
}

// UE8M0 block scale of source/glm_glue.cu:67-74: the exponent byte, scale = 2^(e - 127).
KG_DEV u32 kg_ue8m0(float amax, float eps) {
  const u32 b = kg_f2u(fmaxf(amax, eps) / 448.0f);   // IEEE division (HIP's default is correctly rounded)
  return ((b >> 23) & 0xffu) + ((b & 0x7fffffu) != 0u);
}
KG_DEV float kg_exp2i(u32 e) { return kg_u2f(e << 23); }

// The path's exp (see the file comment).  Evaluated with explicit fmaf so contraction cannot change it.
// Branch-free: the reduction and polynomial run for every x (their value past the range is discarded), and
// the two range tests select at the end, so a wave never splits on them.
KG_DEV float kg_exp(float x) {
  const float xr = fminf(fmaxf(x, -104.0f), 89.0f);          // keeps n and ldexp's exponent finite
  const float n = __builtin_rintf(xr * 1.44269502162933349609375f);
  float r = __builtin_fmaf(n, -0.693145751953125f, x);
  r = __builtin_fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.98412698412698412698e-04f;
  p = __builtin_fmaf(p, r, 1.38888888888888888889e-03f);
  p = __builtin_fmaf(p, r, 8.33333333333333333333e-03f);
  p = __builtin_fmaf(p, r, 4.16666666666666666667e-02f);
  p = __builtin_fmaf(p, r, 1.66666666666666666667e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const float v = __builtin_ldexpf(p, (int)n);            // a NaN x reaches here through r
  return x > 88.72283935546875f ? __builtin_inff() : (x < -103.97208404541015625f ? 0.0f : v);
}

// SiLU(g) = g / (1 + e^-g) for a bf16 gate value g (source/glm_glue.cu:192, whose exp is CUDA's __expf, a
// hardware exp2 of x log2(e)): e^-g as v_exp_f32 of g * -log2(e), the division as g times v_rcp_f32 of
// 1 + e^-g.  Five instructions, two of them transcendental, against about 27 for the Cody-Waite exp and an
// IEEE division; within (|g| log2(e) + 4) f32 ulp of the exact value (the rounding of g * log2(e) scales
// with |g|, as the reference's __expf error does).  The result depends only on g's 16 bits, so the tests
// pin the function as a committed table of its 65536 values, generated on the GPU by this code.
KG_DEV float kg_silu_f32(float g) {
  const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896340736f);
  return g * __builtin_amdgcn_rcpf(1.0f + e);
}

// SiLU(g) * u rounded to bf16 and back (source/glm_glue.cu:192).
KG_DEV float kg_silu_mul_bf16(float g, float u) {
  return kg_bf16_to_f32(kg_f32_to_bf16(kg_silu_f32(g) * u));
}

// The fused epilogue's form of it for two outputs straight from f32 accumulators: the gate and up sums
// rounded to bf16 as the GEMM's bf16 output would hold them, then SiLU(g) * u rounded to bf16 and back.
// The same roundings as kg_silu_mul_bf16 of kg_f32_to_bf16 values, with each pair of them done by one
// v_cvt_pk_bf16_f32 (gate with up, then the two products).
KG_DEV void kg_silu_mul_acc_bf16x2(float g0, float u0, float g1, float u1, float& r0, float& r1) {
  const u32 p0 = kg_pack_bf16x2(g0, u0), p1 = kg_pack_bf16x2(g1, u1);
  const float s0 = kg_silu_f32(kg_u2f(p0 << 16)) * kg_u2f(p0 & 0xffff0000u);
  const float s1 = kg_silu_f32(kg_u2f(p1 << 16)) * kg_u2f(p1 & 0xffff0000u);
  const u32 q = kg_pack_bf16x2(s0, s1);
  r0 = kg_u2f(q << 16);
  r1 = kg_u2f(q & 0xffff0000u);
}

// This lane's id within the wave (v_mbcnt), formed where it is used: the count starts from a zero that an
// empty volatile asm produces at the call, so neither the v_mbcnt pair nor the address arithmetic built on
// it can be hoisted out of a loop into a register held across it (with every register taken, such a value
// is spilled, and its reload waits for all vector memory in flight).  The v_mbcnt instructions themselves
// are the compiler's, so its hazard checks see them.
KG_DEV int kg_lane_here() {
  unsigned z = 0;
  asm volatile("" : "+v"(z));
  return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, z));
}

// Max over groups of `width` consecutive lanes (width a power of two <= 64).
template <int WIDTH>
KG_DEV float kg_group_max(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Max over each row of 16 lanes through DPP (a max does not depend on the pairing): quad permutes [1,0,3,2]
// and [2,3,0,1], then the half-row mirror (lane i <-> 7 - i) and the row mirror (i <-> 15 - i).
template <int CTRL>
KG_DEV float kg_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
KG_DEV float kg_row16_max(float v) {
  v = fmaxf(v, kg_dpp<0xb1>(v));
  v = fmaxf(v, kg_dpp<0x4e>(v));
  v = fmaxf(v, kg_dpp<0x141>(v));
  v = fmaxf(v, kg_dpp<0x140>(v));
  return v;
}
