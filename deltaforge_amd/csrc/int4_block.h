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

// Per-group dequant constants (all exact in fp32: the scale has 8 significant bits, 1032 and
// 72 two set bits each): the scale, -1032 s, s / 16 and -72 s.
struct GroupScale {
  float s, c1, s16, c16;
};

DF_DEVICE GroupScale group_scale(uint16_t sbits) {
  const float s = bf2f(sbits);
  return GroupScale{s, -1032.0f * s, 0.0625f * s, -72.0f * s};
}

// The unpack's masks and fp16 exponent: made once per loop, outside it, and opaque to the
// compiler, so they stay in registers and each unpack is one v_and_or_b32.
struct DqK {
  uint32_t mlo, mhi, bias;
};
DF_DEVICE DqK dq_consts() {
  DqK k{0x000F000Fu, 0x00F000F0u, 0x64006400u};
  asm volatile("" : "+v"(k.mlo), "+v"(k.mhi), "+v"(k.bias));
  return k;
}

typedef _Float16 df_f16x2 __attribute__((ext_vector_type(2)));

// One dword of 8 nibbles -> 8 bf16 weights (4 packed pairs, k order e = 0..7), the reference's
// bf16((nibble - 8) * scale) bit for bit, 17 VALU ops per 8 weights:
//   - one shift and four and-or put each nibble in the mantissa of an fp16 with exponent 2^10:
//     1024 + n for the nibbles at bits 0..3 of a half (e = 0, 1, 4, 5), 1024 + 16 n for those
//     at bits 4..7 (e = 2, 3, 6, 7);
//   - v_fma_mix_f32 widens each fp16 exactly and forms (1024 + n) s - 1032 s, or
//     (1024 + 16 n) (s / 16) - 72 s, with one rounding of an exact value fp32 holds: (n - 8) s
//     exactly (at most 12 significant bits);
//   - v_cvt_pk_bf16_f32 rounds each pair to nearest-even bf16.
DF_DEVICE uint4 dequant8(uint32_t w, const GroupScale& gs, const DqK& K) {
  const uint32_t t = w >> 8;
  const df_f16x2 h0 = __builtin_bit_cast(df_f16x2, (w & K.mlo) | K.bias);  // e0, e1
  const df_f16x2 h1 = __builtin_bit_cast(df_f16x2, (w & K.mhi) | K.bias);  // e2, e3
  const df_f16x2 h2 = __builtin_bit_cast(df_f16x2, (t & K.mlo) | K.bias);  // e4, e5
  const df_f16x2 h3 = __builtin_bit_cast(df_f16x2, (t & K.mhi) | K.bias);  // e6, e7
  const float s = gs.s, c1 = gs.c1, s16 = gs.s16, c16 = gs.c16;
  return make_uint4(pack_bf16(__builtin_fmaf(static_cast<float>(h0.x), s, c1), __builtin_fmaf(static_cast<float>(h0.y), s, c1)),
                    pack_bf16(__builtin_fmaf(static_cast<float>(h1.x), s16, c16), __builtin_fmaf(static_cast<float>(h1.y), s16, c16)),
                    pack_bf16(__builtin_fmaf(static_cast<float>(h2.x), s, c1), __builtin_fmaf(static_cast<float>(h2.y), s, c1)),
                    pack_bf16(__builtin_fmaf(static_cast<float>(h3.x), s16, c16), __builtin_fmaf(static_cast<float>(h3.y), s16, c16)));
}

}  // namespace df
