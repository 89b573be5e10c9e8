// Device decoders of one 256-element unit of a GGUF-block weight row in the
// panel layout of QLinearKQ ([panel][block][plane][64 rows][16 B], kquant.hip
// upload): the lane is the row, the activations are the same for every lane
// (a broadcast operand from LDS or a scalar load), and each function adds
// sum_k w_k x_k of its unit to `acc`.
//
// Q4_K / Q6_K use mixed-precision FMAs (v_fma_mix_f32: f16 weight operand,
// f32 activation and accumulator).  Quant fields masked in place inside the
// low 8 bits of a 16-bit half are exact f16 subnormals q * 2^-24 times a
// power of two set by their bit offset, so each element costs one FMA and a
// few masks per dword instead of an extract, a convert and an FMA:
//   nibbles (Q4_K, Q6_K low bits), element k at bits 4k of a dword:
//     w & 0x000f000f -> (e0, e4)   w & 0x00f000f0 -> 16 (e1, e5)   (w>>8): (e2,e6), 16 (e3,e7)
//   Q6_K: each ql dword's nibbles joined in place with their two-bit qh
//     fields (the two qh bytes spread to the two halves, one byte permute),
//     so the six-bit value lo + 16 hi of a pair of elements is one masked
//     dword of class 1 or 16 and each element still costs one FMA
// Each power-of-two class has its own f32 accumulator; the classes are
// combined with exact power-of-two FMAs, so the values are the f32 path's
// (up to summation order).  Sub-block sums of the activations (`as`: Q4_K's
// dmin term per 32 elements, Q6_K's -32 offset per 16) come from the caller.
#pragma once

#include "common.hpp"

namespace syn {

typedef _Float16 kq_h2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ kq_h2 kq_as_h2(uint32_t v) { return __builtin_bit_cast(kq_h2, v); }

// sum_k e_k x_k over the 8 nibbles of w, scaled by 2^-24: returns into
// a (class x1) and b (class x16)
__device__ __forceinline__ void kq_nib8(uint32_t w, const float *__restrict__ xc, float &a,
                                        float &b) {
  const uint32_t w8 = w >> 8;
  const kq_h2 p0 = kq_as_h2(w & 0x000f000fu), p1 = kq_as_h2(w & 0x00f000f0u);
  const kq_h2 p2 = kq_as_h2(w8 & 0x000f000fu), p3 = kq_as_h2(w8 & 0x00f000f0u);
  a = __builtin_fmaf((float)p0.x, xc[0], a);
  b = __builtin_fmaf((float)p1.x, xc[1], b);
  a = __builtin_fmaf((float)p2.x, xc[2], a);
  b = __builtin_fmaf((float)p3.x, xc[3], b);
  a = __builtin_fmaf((float)p0.y, xc[4], a);
  b = __builtin_fmaf((float)p1.y, xc[5], b);
  a = __builtin_fmaf((float)p2.y, xc[6], a);
  b = __builtin_fmaf((float)p3.y, xc[7], b);
}

// Q4_K superblock (gguf.rs:375-438): pl[0] = f16 d | f16 dmin | 12 scale
// bytes, pl[1 + s] = the 32 nibbles of sub-block s.  Stage sb adds sub-block
// sb: xc = its 32 activations, as = their sum.
__device__ __forceinline__ void kq4_stage(const u32x4 *pl, int sb, float d, float dmin,
                                          const float *__restrict__ xc, float as, float &acc) {
  const uint32_t sbw[3] = {pl[0].y, pl[0].z, pl[0].w};
  auto SB = [&](int i) -> uint32_t { return (sbw[i >> 2] >> (8 * (i & 3))) & 0xffu; };
  uint32_t sc, mn;  // gguf.rs:405-410, u8 arithmetic
  if (sb < 4) {
    sc = SB(sb) & 63u;
    mn = ((SB(sb + 4) >> 4) | ((SB(sb + 8) & 15u) << 4)) & 0xffu;
  } else {
    sc = (SB(sb) & 15u) | ((SB(sb - 4) >> 6) << 4);
    mn = ((SB(sb + 4) >> 4) | (((SB(sb - 4) >> 4) & 12u) << 4)) & 0xffu;
  }
  const float scf = d * (float)sc;
  const float mf = dmin * (float)mn;
  const u32x4 q = pl[1 + sb];
  float a = 0.0f, c16 = 0.0f;
  kq_nib8(q.x, xc, a, c16);
  kq_nib8(q.y, xc + 8, a, c16);
  kq_nib8(q.z, xc + 16, a, c16);
  kq_nib8(q.w, xc + 24, a, c16);
  const float t = __builtin_fmaf(c16, 0.0625f, a) * 16777216.0f;
  acc = __builtin_fmaf(scf, t, acc);
  acc = __builtin_fmaf(-mf, as, acc);
}

__device__ __forceinline__ void kq4_unit(const u32x4 *pl, const float *__restrict__ xs,
                                         const float *__restrict__ as, float &acc) {
  const float d = syn_f16_to_f32_rs(pl[0].x & 0xffffu);
  const float dmin = syn_f16_to_f32_rs(pl[0].x >> 16);
#pragma unroll
  for (int sb = 0; sb < 8; sb++) kq4_stage(pl, sb, d, dmin, xs + sb * 32, as[sb], acc);
}

// Q6_K superblock (gguf.rs:440-487): pl[0..7] = ql (128 B), pl[8..11] = qh
// (64 B), pl[12] = 16 int8 scales, d = the f16 d.  Group g: 16 elements,
// xc = its activations, as = their sum.
__device__ __forceinline__ void kq6_group(const u32x4 *pl, int g, float d,
                                          const float *__restrict__ xc, float as, float &acc) {
  const uint32_t scw[4] = {pl[12].x, pl[12].y, pl[12].z, pl[12].w};
  // ql bytes 8g..8g+7: plane g/2, dwords 2*(g%2), 2*(g%2)+1
  const u32x4 qp = pl[g >> 1];
  const uint32_t lo0 = (g & 1) ? qp.z : qp.x, lo1 = (g & 1) ? qp.w : qp.y;
  // qh bytes 4g..4g+3: plane 8 + g/4, dword g%4
  const u32x4 hp = pl[8 + (g >> 2)];
  const uint32_t hi = (g & 3) == 0 ? hp.x : (g & 3) == 1 ? hp.y : (g & 3) == 2 ? hp.z : hp.w;
  const float scale = (float)(int8_t)(scw[g >> 2] >> (8 * (g & 3))) * d;
  // the six-bit value lo + 16 hi assembled in place: for the eight elements
  // of one ql dword L (nibble of element i at bits 4i), H = the two qh bytes
  // of those elements in the two 16-bit halves (field of element i at bits
  // 2(i % 4) of its half); each pair (i, i + 4) then sits in one dword as
  // two f16 subnormals of class 1 (bits 0-5) or 16 (bits 4-9)
  float a1 = 0.0f, a16 = 0.0f;
#pragma unroll
  for (int half = 0; half < 2; half++) {
    const uint32_t L = half ? lo1 : lo0, L8 = L >> 8;
    const uint32_t hb = half ? hi >> 16 : hi;
    const uint32_t H = (hb & 0xffu) | ((hb << 8) & 0x00ff0000u);
    const kq_h2 p0 = kq_as_h2((L & 0x000f000fu) | ((H << 4) & 0x00300030u));   // (e0, e4) x1
    const kq_h2 p1 = kq_as_h2((L & 0x00f000f0u) | ((H << 6) & 0x03000300u));   // (e1, e5) x16
    const kq_h2 p2 = kq_as_h2((L8 & 0x000f000fu) | (H & 0x00300030u));         // (e2, e6) x1
    const kq_h2 p3 = kq_as_h2((L8 & 0x00f000f0u) | ((H << 2) & 0x03000300u));  // (e3, e7) x16
    const float *x = xc + 8 * half;
    a1 = __builtin_fmaf((float)p0.x, x[0], a1);
    a16 = __builtin_fmaf((float)p1.x, x[1], a16);
    a1 = __builtin_fmaf((float)p2.x, x[2], a1);
    a16 = __builtin_fmaf((float)p3.x, x[3], a16);
    a1 = __builtin_fmaf((float)p0.y, x[4], a1);
    a16 = __builtin_fmaf((float)p1.y, x[5], a16);
    a1 = __builtin_fmaf((float)p2.y, x[6], a1);
    a16 = __builtin_fmaf((float)p3.y, x[7], a16);
  }
  const float t = __builtin_fmaf(a16, 0.0625f, a1) * 16777216.0f;
  const float v = t - 32.0f * as;
  acc = __builtin_fmaf(v, scale, acc);
}

__device__ __forceinline__ void kq6_unit(const u32x4 *pl, uint16_t dh, const float *__restrict__ xs,
                                         const float *__restrict__ as, float &acc) {
  const float d = syn_f16_to_f32_rs(dh);
#pragma unroll
  for (int g = 0; g < 16; g++) kq6_group(pl, g, d, xs + g * 16, as[g], acc);
}

// Q8_0 block j of a unit of eight (gguf.rs:255-288): pl[2j], pl[2j+1] = its
// 32 int8, d = its f16 d, xc = its 32 activations
__device__ __forceinline__ void kq8_block(const u32x4 *pl, int j, float d,
                                          const float *__restrict__ xc, float &acc) {
  const uint32_t q[8] = {pl[2 * j].x,     pl[2 * j].y,     pl[2 * j].z,     pl[2 * j].w,
                         pl[2 * j + 1].x, pl[2 * j + 1].y, pl[2 * j + 1].z, pl[2 * j + 1].w};
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int b = 0; b < 4; b++)
      s = __builtin_fmaf(xc[4 * i + b], (float)(int8_t)(q[i] >> (8 * b)), s);
  acc = __builtin_fmaf(s, d, acc);
}

// Q4_0 block (one 16-byte plane: element 2i in the low nibble of byte i,
// 2i+1 in the high; value (q - 8) * d): the nibbles as in-place f16
// subnormals (the masks above), s0 over the even elements at 2^-24, s1 over
// the odd at 16 * 2^-24, then the -8 offset as 8 * xsum (the caller's sum of
// the block's 32 activations).
__device__ __forceinline__ void kq40_block(const u32x4 &pl, float d, const float *__restrict__ xc,
                                           float xsum, float &acc) {
  const uint32_t wd[4] = {pl.x, pl.y, pl.z, pl.w};
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const uint32_t w = wd[c], w8 = wd[c] >> 8;
    const float *x = xc + 8 * c;
    const kq_h2 p0 = kq_as_h2(w & 0x000f000fu), p1 = kq_as_h2(w & 0x00f000f0u);
    const kq_h2 p2 = kq_as_h2(w8 & 0x000f000fu), p3 = kq_as_h2(w8 & 0x00f000f0u);
    s0 = __builtin_fmaf((float)p0.x, x[0], s0);
    s1 = __builtin_fmaf((float)p1.x, x[1], s1);
    s0 = __builtin_fmaf((float)p2.x, x[2], s0);
    s1 = __builtin_fmaf((float)p3.x, x[3], s1);
    s0 = __builtin_fmaf((float)p0.y, x[4], s0);
    s1 = __builtin_fmaf((float)p1.y, x[5], s1);
    s0 = __builtin_fmaf((float)p2.y, x[6], s0);
    s1 = __builtin_fmaf((float)p3.y, x[7], s1);
  }
  const float dot = __builtin_fmaf(s1, 0.0625f, s0) * 16777216.0f;
  acc = __builtin_fmaf(dot - 8.0f * xsum, d, acc);
}

}  // namespace syn
