// Host exact tier of libexactattn_hip.so (ea_exact_host.cpp): one attention row computed with
// exact integer arithmetic on the CPU. The device tiers (tier 1 on the kernels, tier 2 in 128-bit
// windows) certify every row the benchmarks and the reference's fixtures hold; a row they leave
// uncertified (flag 1: massive cancellation in a numerator, a score whose 120-bit window cannot
// decide its logit, an exp2 that 128 bits cannot round) is recomputed here, exactly, and counted.
// Reference counterpart: the host recompute of flagged rows, reference.attention_row
// (src/exactattn/reference.py:82-147) called from src/exactattn/cpu.py:105-108 and
// src/exactattn/triton_kernels.py:1556-1559.
#pragma once
#include <stdint.h>

namespace eax {

// Result codes of exact_row.
enum { EAX_OK = 0, EAX_DOMAIN = 2, EAX_REFUSED = 3, EAX_NOMEM = 4 };

// Per-key intermediates of a row (optional output of exact_row): t = RN32(alpha s) as fp32 bits,
// w = RN24(2^t) = wm 2^we (we saturates at +-2^62 for logits beyond that range).
struct KeyTrace {
    uint32_t* t_bits;
    int32_t* wm;
    int64_t* we;
};

// q: d bf16 bit patterns; K: n rows of d, V: n rows of dv (row-major, contiguous); alpha as fp32
// bits; out: dv bf16 (uint16) or fp32 (uint32) bit patterns, +0 for zero. Returns EAX_OK,
// EAX_DOMAIN for a NaN/inf input or an fp32 logit overflow (out untouched), or EAX_REFUSED when
// deciding a rounding would need the exact sums over an exponent spread above 2^20 bits (the
// reference's own limit, src/exactattn/reference.py:27-30), or EAX_NOMEM when the host heap is
// exhausted (no exception leaves this function).
int exact_row(const uint16_t* q, int d, const uint16_t* K, const uint16_t* V, int64_t n, int dv, uint32_t alpha_bits,
              int fp32, void* out, const KeyTrace* tr) noexcept;

// RN-even of (a / b) * 2^E with a, b given as 128-bit (hi, lo) words, b > 0, into fp32 (p = 24)
// or bf16 (p = 8) with gradual underflow. Returns the result's bit pattern (negated when neg) and
// sets *overflow when it exceeds the format's largest finite value (bits are then 0).
uint32_t round_ratio_bits(uint64_t a_hi, uint64_t a_lo, uint64_t b_hi, uint64_t b_lo, int64_t E, int neg, int fp32,
                          int* overflow) noexcept;

}  // namespace eax
