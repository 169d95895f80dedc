// INT8 quantisation helpers shared by the quantisation kernels and the
// pooling pass that quantises Q (compiled with -ffp-contract=off: every fp32
// operation is rounded where it is written).
//
// Codes are trunc(fl(q + copysign(0.5, q))) of the IEEE quotient q = fl(x / s),
// clamped to [-127, 127], exactly as the CPU oracle rounds. The kernels form
// q' = x * rcp(s) instead (v_rcp_f32, within 1 ulp of 1/s), within 2 ulp of q
// (|q| <= 127 * (1 + 2^-22), so an ulp is at most 7.6e-6), and v = fl(q' + 128)
// within 2.3e-5 of q + 128. When v lies farther than kNearTie = 4e-5 from every
// half-integer, q + 128 and v round to the same nearest integer and
// fl(q + copysign(0.5, q)) stays clear of every integer, so the code is
// rint(v) - 128: v_cvt_pk_u8_f32 (round to nearest) writes rint(v) into a byte
// and an XOR with 0x80 per byte subtracts the 128. A lane holding a value within
// kNearTie of a half-integer recomputes its eight codes by IEEE division.
#pragma once

#include "common.hpp"

namespace solattn {

// Low bytes of four ints -> one dword (v_perm_b32: selector 0-3 picks a byte
// of the second operand, 4-7 of the first, 12 gives 0x00).
__device__ __forceinline__ uint32_t pack_i8x4(int a, int b, int c, int d) {
  const uint32_t ab = __builtin_amdgcn_perm(static_cast<uint32_t>(b), static_cast<uint32_t>(a),
                                            0x0c0c0400u);  // a0 b0 0 0
  const uint32_t cd = __builtin_amdgcn_perm(static_cast<uint32_t>(d), static_cast<uint32_t>(c),
                                            0x0c0c0400u);  // c0 d0 0 0
  return __builtin_amdgcn_perm(cd, ab, 0x05040100u);      // a0 b0 c0 d0
}

// t = fl(q + copysign(0.5, q)) -> trunc(t) clamped to [-127, 127]
// (v_cvt_i32_f32 truncates).
__device__ __forceinline__ int code_of(float t) {
  return static_cast<int>(__builtin_amdgcn_fmed3f(t, -127.f, 127.f));
}

// |v - rint(v)|, in [0, 0.5]: v is within kNearTie of a half-integer when
// this is >= 0.5 - kNearTie.
__device__ __forceinline__ float int_distance(float v) { return fabsf(v - __builtin_rintf(v)); }
constexpr float kNearTie = 4e-5f;

// fl(a / 127) for a >= 0 without a division: q0 = a * fl(1/127) corrected by
// one fma residual step. Equal to the IEEE quotient for every non-negative
// finite float (checked exhaustively on the CPU, tests/test_oracle.py).
__device__ __forceinline__ float div127(float a) {
  const float c = 1.0f / 127.0f;
  const float q0 = a * c;
  const float r = __builtin_fmaf(-q0, 127.0f, a);
  return __builtin_fmaf(r, c, q0);
}

// Max over the 16 lanes of a lane group through DPP lane moves (no LDS):
// swap neighbours, swap pairs, mirror within 8 lanes, mirror within 16. On
// the bit patterns of non-negative floats, whose unsigned order is their
// numeric order.
__device__ __forceinline__ uint32_t group16_max_bits(uint32_t x) {
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0xB1, 0xf, 0xf, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x4E, 0xf, 0xf, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x141, 0xf, 0xf, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x140, 0xf, 0xf, false)));
  return x;
}

// Codes of eight values against one reciprocal scale rr = rcp(s) (or eight),
// re-derived by IEEE division by s when any lies near a rounding tie.
__device__ __forceinline__ uint2 codes8(const float (&y)[8], const float (&rr)[8],
                                        const float (&s)[8]) {
  uint32_t lo = 0u, hi = 0u;
  float d = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float v = y[e] * rr[e] + 128.f;  // fl(fl(y * rr) + 128) (no contraction here)
    d = fmaxf(d, int_distance(v));
    if (e < 4) lo = __builtin_amdgcn_cvt_pk_u8_f32(v, e, lo);
    else hi = __builtin_amdgcn_cvt_pk_u8_f32(v, e - 4, hi);
  }
  if (d >= 0.5f - kNearTie) {
    asm volatile("");  // keeps the divisions on this rare path
    int code[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float q = y[e] / s[e];
      code[e] = code_of(q + copysignf(0.5f, q));
    }
    return make_uint2(pack_i8x4(code[0], code[1], code[2], code[3]),
                      pack_i8x4(code[4], code[5], code[6], code[7]));
  }
  return make_uint2(lo ^ 0x80808080u, hi ^ 0x80808080u);
}

// Per-token INT8 of one row held by a 16-lane group, 8 channels per lane
// (y already smoothed): the row scale s = max(fl(max|y| / 127), 1e-8) and
// this lane's 8 codes packed into two dwords. max|y| by float compares (the
// same value as on bit patterns for every non-NaN row).
__device__ __forceinline__ float quant_token_row(const float (&y)[8], uint2& packed) {
  const float m4 = fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3])));
  const float m8 = fmaxf(m4, fmaxf(fmaxf(fabsf(y[4]), fabsf(y[5])), fmaxf(fabsf(y[6]), fabsf(y[7]))));
  const float sc = div127(__uint_as_float(group16_max_bits(__float_as_uint(m8))));
  const float ss = sc > 1e-8f ? sc : 1e-8f;
  const float r = __builtin_amdgcn_rcpf(ss);
  const float rr[8] = {r, r, r, r, r, r, r, r}, sv[8] = {ss, ss, ss, ss, ss, ss, ss, ss};
  packed = codes8(y, rr, sv);
  return ss;
}

}  // namespace solattn
