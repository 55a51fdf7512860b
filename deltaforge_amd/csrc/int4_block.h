// The int4 device tiling and its exact dequant, shared by the GEMV and the persistent
// decode kernel.
//
//   block (t, g) = 1024 bytes for output columns 16t..16t+15 and k in group g
//                = [slot s 0..3][column c 0..15][16 bytes]
//   16 bytes     = 4 dwords d; dword d holds k = 128g + 32s + 8d + e, e = 0..7, with
//                  nibble e=2j at bits 4j..4j+3 and e=2j+1 at bits 16+4j..16+4j+3.
//   blocks are ordered [t][g]; scales are [t][g][16] bf16.
#pragma once

#include "common.h"

namespace df {

constexpr int kGroup = 128;
constexpr int kTileCols = 16;
constexpr int kBlockBytes = 1024;

typedef __bf16 df_bf16x2 __attribute__((ext_vector_type(2)));
typedef float df_f32x2 __attribute__((ext_vector_type(2)));

DF_DEVICE uint4 load16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

DF_DEVICE uint32_t pack_bf16(float a, float b) {
  const df_f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, df_bf16x2));
}

// Per-group dequant constants: 512 * scale and -8 * scale (both exact in fp32).
struct GroupScale {
  float s512, neg8s;
};

DF_DEVICE GroupScale group_scale(uint16_t sbits) {
  const float s = bf2f(sbits);
  return GroupScale{512.0f * s, -8.0f * s};
}

// w & 0x0F0F0F0F as one opaque instruction, so the byte conversions below stay
// v_cvt_f32_ubyte{0..3} of the masked word instead of one bit-field extract per nibble.
// (Only plain ALU ops go through inline asm: the compiler cannot see the issue latency of an
// instruction it only knows as text, so anything whose result needs wait states stays in C.)
DF_DEVICE uint32_t low_nibbles(uint32_t w) {
  uint32_t r;
  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(w));
  return r;
}

// One dword of 8 nibbles -> 8 bf16 weights (4 packed pairs, k order e = 0..7).
// A byte holding a nibble n (0..15) is the OCP E4M3 encoding of n * 2^-9 (subnormal for
// n < 8, exponent field 1 for n >= 8, linear across the boundary), so v_cvt_pk_f32_fp8 turns
// two nibbles into two exact floats per instruction; fma(n 2^-9, 512 s, -8 s) = (n - 8) s
// exactly (at most 12 significant bits) and v_cvt_pk_bf16_f32 rounds each pair to
// nearest-even bf16: the reference's bf16((nibble - 8) * scale). 19 VALU ops per 8 weights.
DF_DEVICE uint4 dequant8(uint32_t w, const GroupScale& gs) {
  const uint32_t lo = low_nibbles(w);       // bytes: e0, e4, e1, e5
  const uint32_t hi = low_nibbles(w >> 4);  // bytes: e2, e6, e3, e7
  const df_f32x2 f04 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(lo), false);
  const df_f32x2 f15 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(lo), true);
  const df_f32x2 f26 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(hi), false);
  const df_f32x2 f37 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(hi), true);
  const float s = gs.s512, c = gs.neg8s;
  const float e0 = __builtin_fmaf(f04.x, s, c), e4 = __builtin_fmaf(f04.y, s, c);
  const float e1 = __builtin_fmaf(f15.x, s, c), e5 = __builtin_fmaf(f15.y, s, c);
  const float e2 = __builtin_fmaf(f26.x, s, c), e6 = __builtin_fmaf(f26.y, s, c);
  const float e3 = __builtin_fmaf(f37.x, s, c), e7 = __builtin_fmaf(f37.y, s, c);
  return make_uint4(pack_bf16(e0, e1), pack_bf16(e2, e3), pack_bf16(e4, e5), pack_bf16(e6, e7));
}

}  // namespace df
