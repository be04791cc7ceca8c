// Operand maps of the bit-exact batched GEMM (uq_gemm_q8k.hip), shared by
// the kernel and its host emulation (uq_emu.cpp).
//
// gemv_quant_q8k sums, per row and 256-block, eight integer lane sums
// sumi[k] = sum over the elements e with e % 8 == k of sc(e) * q(e) * q8(e)
// (dot_q4_k_q8_k quants.rs:337-342, dot_q6_k_q8_k :390-401). The GEMM forms
// each lane sum on the f16 MFMA: the 32 elements e = 8 j + l of lane l are
// the K of two 16-deep MFMAs (j in [16 h, 16 h + 16) for h = 0, 1), every
// operand an exact f16 integer (|q8| <= 127; Q4_K sc*q <= 945; Q6_K the
// exact pair (sc & ~1)*q, (sc & 1)*q, |.| <= 4096) and every partial sum an
// integer below 2^24, so the f32 accumulation is exact in any order.
//
// An MFMA operand holds, per lane, one k-octet: 8 of the 16 j of its half
// h. Octet (l, h, o) of a block and its slot s (0..7) name one element;
// the activation side writes q8 of that element into the slot, the weight
// side decodes the same element's weight into it. The slot order follows
// what the weight decode produces cheaply, and differs per format:
//   Q4_K  octet (l, h, o) is qs chunk c = 2h + o (groups 2c and 2c+1): the
//         four bytes 32c + 8i + l (i = 0..3), low nibbles then high;
//         j = 16h + 8o + 4(s >> 2) + t(s).
//   Q6_K  octet (l, h, o) is the four ql bytes 64h + 32o + 8i + l, low
//         nibbles (elements 128h + 32o + 8i + l) then high (+64), each with
//         its 2-bit field of qh byte 32h + 8i + l;
//         j = 16h + 8(s >> 2) + 4o + t(s).
// with t(s) = (0, 2, 1, 3)[s & 3]: an f16 pair is bytes (0, 2) or (1, 3)
// of a dword (bit-field insert into the mantissa of 1024).
#pragma once

#include "uq_bits.h"

namespace uq {

// Element (0..255) of slot s of octet (l, h, o).
template <bool Q6>
UQ_HD int q8k_slot_elem(int l, int h, int o, int s) {
    const int t = ((s & 1) << 1) | ((s >> 1) & 1);
    const int j = Q6 ? 16 * h + 8 * (s >> 2) + 4 * o + t : 16 * h + 8 * o + 4 * (s >> 2) + t;
    return 8 * j + l;
}

// scale_min_k4 (quants.rs:92-102): the 6-bit scale and min of Q4_K group g
// from the block's scale dwords S0 = s[0..3], S1 = s[4..7], S2 = s[8..11].
UQ_HD uint32_t q4k_sc(uint32_t S0, uint32_t S2, int g) {
    return g < 4 ? (S0 >> (8 * g)) & 63 : ((S2 >> (8 * (g - 4))) & 0xF) | (((S0 >> (8 * (g - 4) + 6)) & 3) << 4);
}
UQ_HD uint32_t q4k_m(uint32_t S1, uint32_t S2, int g) {
    return g < 4 ? (S1 >> (8 * g)) & 63 : ((S2 >> (8 * (g - 4) + 4)) & 0xF) | (((S1 >> (8 * (g - 4) + 6)) & 3) << 4);
}

// v_bfi_b32: (x & mask) | (y & ~mask)
UQ_HD uint32_t bfi32(uint32_t mask, uint32_t x, uint32_t y) {
#if defined(__HIP_DEVICE_COMPILE__)
    uint32_t r;
    __asm__("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(mask), "v"(x), "v"(y));
    return r;
#else
    return (x & mask) | (y & ~mask);
#endif
}

// The four dwords of byte lane l (0..7) of a 32-byte run w[0..7] of raw
// bytes at stride 8: run bytes l, 8 + l, 16 + l, 24 + l are the transposes
// of w[l/4 + 2i], i = 0..3 (t[l % 4] of q8k_gather; transpose4 is the
// 4x4 byte transpose of uq_bits.h).
UQ_HD void q8k_gather(const uint32_t w[8], int lg, uint32_t (&t)[4]) {
    transpose4(w[lg], w[lg + 2], w[lg + 4], w[lg + 6], t);
}

// Q4_K octet from its gathered dword T (bytes 32c + 8i + l, i = 0..3): four
// f16 pairs (bit patterns), slots (0,1) (2,3) (4,5) (6,7):
//   1024 + nibble of bytes (0, 2), (1, 3) low nibbles,
//   1024 + 16 * nibble of bytes (0, 2), (1, 3) high nibbles.
// fma(p, sc, -1024 sc) and fma(p, sc / 16, -64 sc) give sc * nibble exactly.
UQ_HD void q4k_pairs(uint32_t T, uint32_t p[4]) {
    const uint32_t lm = 0x000F000Fu, hm = 0x00F000F0u, mag = 0x64006400u, T8 = T >> 8;
    p[0] = bfi32(lm, T, mag);
    p[1] = bfi32(lm, T8, mag);
    p[2] = bfi32(hm, T, mag);
    p[3] = bfi32(hm, T8, mag);
}

// Q6_K raw 6-bit values of an octet: QL the gathered ql bytes
// (64h + 32o + 8i + l), QH the gathered qh bytes (32h + 8i + l). Low
// nibbles take qh bits 2o..2o+1 (element 128h + 32o + 8i + l), high nibbles
// bits 2o+4..2o+5 (element + 64): ra / rb hold raw (0..63) per byte.
UQ_HD void q6k_raw(uint32_t QL, uint32_t QH, int o, uint32_t &ra, uint32_t &rb) {
    const uint32_t qs = QH >> (2 * o);
    ra = (QL & 0x0F0F0F0Fu) | ((qs << 4) & 0x30303030u);
    rb = ((QL >> 4) & 0x0F0F0F0Fu) | (qs & 0x30303030u);
}

// 1024 + raw of bytes (0, 2) and (1, 3) of r as f16 pairs; raw - 32 = q is
// the pair minus 1056, exact.
UQ_HD void q6k_pairs(uint32_t r, uint32_t p[2]) {
    const uint32_t bm = 0x00FF00FFu, mag = 0x64006400u;
    p[0] = bfi32(bm, r, mag);
    p[1] = bfi32(bm, r >> 8, mag);
}

}  // namespace uq
