// INT8 quantisation helpers shared by the quantisation kernels and the
// pooling pass that quantises Q (compiled with -ffp-contract=off: every fp32
// operation is rounded where it is written).
//
// Codes are trunc(fl(q + copysign(0.5, q))) of the IEEE quotient q = fl(x / s),
// clamped to [-127, 127], exactly as the CPU oracle rounds. The kernels form
// q' = x * rcp(s) instead (v_rcp_f32, within 1 ulp of 1/s), within 2 ulp of q;
// trunc(fl(. + 0.5)) can only differ between q and q' when fl(q' + 0.5) lies
// within 4e-5 of an integer (|q| <= 127.5, so an ulp is at most 7.7e-6), and a
// lane holding such a value recomputes its eight codes by IEEE division.
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

// |t - rint(t)|: a code is re-derived by division when this is <= kNearTie.
__device__ __forceinline__ float tie_distance(float t) { return fabsf(t - __builtin_rintf(t)); }
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
  int code[8];
  float d = 1.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float q1 = y[e] * rr[e];
    const float tq = q1 + copysignf(0.5f, q1);
    d = fminf(d, tie_distance(tq));
    code[e] = code_of(tq);
  }
  if (d <= kNearTie) {
    asm volatile("");  // keeps the divisions on this rare path
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float q = y[e] / s[e];
      code[e] = code_of(q + copysignf(0.5f, q));
    }
  }
  return make_uint2(pack_i8x4(code[0], code[1], code[2], code[3]),
                    pack_i8x4(code[4], code[5], code[6], code[7]));
}

// Per-token INT8 of one row held by a 16-lane group, 8 channels per lane
// (y already smoothed): the row scale s = max(fl(max|y| / 127), 1e-8) and
// this lane's 8 codes packed into two dwords.
__device__ __forceinline__ float quant_token_row(const float (&y)[8], uint2& packed) {
  uint32_t m = 0;  // max |y| as bits
#pragma unroll
  for (int e = 0; e < 8; ++e) m = max(m, __float_as_uint(y[e]) & 0x7fffffffu);
  const float sc = div127(__uint_as_float(group16_max_bits(m)));
  const float ss = sc > 1e-8f ? sc : 1e-8f;
  const float r = __builtin_amdgcn_rcpf(ss);
  const float rr[8] = {r, r, r, r, r, r, r, r}, sv[8] = {ss, ss, ss, ss, ss, ss, ss, ss};
  packed = codes8(y, rr, sv);
  return ss;
}

}  // namespace solattn
