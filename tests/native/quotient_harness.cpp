// Host build of the library's quotient rounding (exactattention_amd/csrc/ea_quotient.h, the code
// the tier-2 kernel runs), for tests/test_quotient.py: plain C entry points over ctypes.
#include <stdint.h>

#include "../../exactattention_amd/csrc/ea_quotient.h"

using ea::i128;
using ea::u128;

static i128 s128(int64_t hi, uint64_t lo) { return (i128)(((u128)(uint64_t)hi << 64) | lo); }

extern "C" int h_rn_quotient(uint64_t a_hi, uint64_t a_lo, uint64_t b_hi, uint64_t b_lo, int64_t sh, int fp32,
                             uint32_t* Q, int32_t* qe) {
    ea::quant y;
    const int st = ea::rn_quotient(((u128)a_hi << 64) | a_lo, ((u128)b_hi << 64) | b_lo, sh, fp32 ? 24 : 8,
                                   fp32 ? -149 : -133, &y);
    *Q = y.Q;
    *qe = y.qe;
    return st;
}

// v: Nlo, Nhi, Zlo, Zhi as (hi, lo) pairs of words, then sh. Returns 1 when certified.
extern "C" int h_certify_quotient(const int64_t* v, int fp32, uint32_t* bits) {
    *bits = 0xFFFFFFFFu;
    return ea::certify_quotient(s128(v[0], (uint64_t)v[1]), s128(v[2], (uint64_t)v[3]), s128(v[4], (uint64_t)v[5]),
                                s128(v[6], (uint64_t)v[7]), v[8], fp32, bits)
               ? 1
               : 0;
}

extern "C" uint32_t h_fmt_bits(uint32_t Q, int qe, int neg, int fp32) { return ea::fmt_bits(Q, qe, neg != 0, fp32); }
