// Exact rounding of a quotient to bf16 or fp32: tier 2's certified final rounding, and the
// format encoder rn32_prod shares. Plain integer and fp64 code, compiled for the device (the
// kernels) and for the host (a CPU test builds this same header with g++ and checks it against
// exact rationals).
#pragma once
#include <math.h>
#include <stdint.h>

#if defined(__HIPCC__)
#define EA_HD __host__ __device__
#else
#define EA_HD
#endif

namespace ea {

typedef __int128 i128;
typedef unsigned __int128 u128;

EA_HD inline int q_bitlen128(u128 x) {
    const uint64_t hi = (uint64_t)(x >> 64), lo = (uint64_t)x;
    return hi ? 128 - __builtin_clzll(hi) : (lo ? 64 - __builtin_clzll(lo) : 0);
}

// ------------------------------------------------------------------------------------------------
// Exact rounding of a quotient (tier 2's final rounding; the format encoder is shared with
// rn32_prod). Values are Q * 2^qe with Q < 2^p, Q >= 2^(p-1) unless qe = qmin (subnormal or
// zero). Three-word integers (192 bits) hold every product formed here: a numerator below 2^127
// scaled by at most the precision plus a few bits, or a denominator below 2^127 times a multiple
// below 2^27.
// ------------------------------------------------------------------------------------------------
struct w192 {
    uint64_t w0, w1, w2;
};

// x * 2^s for s >= 0 and bitlen(x) + s <= 192
EA_HD inline w192 w192_shifted(u128 x, int s) {
    const uint64_t lo = (uint64_t)x, hi = (uint64_t)(x >> 64);
    w192 r = {0, 0, 0};
    if (s >= 128) {
        r.w2 = lo << (s - 128);
    } else if (s >= 64) {
        const int t = s - 64;
        r.w1 = lo << t;
        r.w2 = t ? (hi << t) | (lo >> (64 - t)) : hi;
    } else {
        r.w0 = lo << s;
        r.w1 = s ? (hi << s) | (lo >> (64 - s)) : hi;
        r.w2 = s ? hi >> (64 - s) : 0;
    }
    return r;
}
EA_HD inline w192 w192_shl(const w192& a, int s) {  // s in [0, 64), no bits lost
    if (!s) return a;
    return {a.w0 << s, (a.w1 << s) | (a.w0 >> (64 - s)), (a.w2 << s) | (a.w1 >> (64 - s))};
}
EA_HD inline w192 w192_shl_any(w192 a, int s) {  // s in [0, 192), no bits lost
    for (; s >= 64; s -= 64) a = {0, a.w0, a.w1};
    return w192_shl(a, s);
}
EA_HD inline int w192_cmp(const w192& a, const w192& b) {
    if (a.w2 != b.w2) return a.w2 < b.w2 ? -1 : 1;
    if (a.w1 != b.w1) return a.w1 < b.w1 ? -1 : 1;
    if (a.w0 != b.w0) return a.w0 < b.w0 ? -1 : 1;
    return 0;
}
EA_HD inline w192 w192_sub(const w192& a, const w192& b) {  // a >= b
    const uint64_t r0 = a.w0 - b.w0, c0 = a.w0 < b.w0;
    const uint64_t t1 = a.w1 - b.w1, c1 = a.w1 < b.w1;
    const uint64_t r1 = t1 - c0, c1b = t1 < c0;
    return {r0, r1, a.w2 - b.w2 - c1 - c1b};
}
EA_HD inline w192 w192_add(const w192& a, const w192& b) {
    const uint64_t r0 = a.w0 + b.w0, c0 = r0 < a.w0;
    const uint64_t t1 = a.w1 + b.w1, c1 = t1 < a.w1;
    const uint64_t r1 = t1 + c0, c1b = r1 < t1;
    return {r0, r1, a.w2 + b.w2 + c1 + c1b};
}
// a * m for a < 2^160, m < 2^32
EA_HD inline w192 w192_mul32(const w192& a, uint32_t m) {
    const u128 p0 = (u128)a.w0 * m;
    const u128 p1 = (u128)a.w1 * m + (uint64_t)(p0 >> 64);
    return {(uint64_t)p0, (uint64_t)p1, a.w2 * m + (uint64_t)(p1 >> 64)};
}
// a rounded to fp64 (relative error below 2^-52): the leading 64 bits, converted, then scaled
EA_HD inline double w192_f64(const w192& a) {
    if (a.w2) {
        const int z = __builtin_clzll(a.w2);
        const uint64_t top = z ? (a.w2 << z) | (a.w1 >> (64 - z)) : a.w2;
        return ldexp((double)top, 128 - z);
    }
    if (a.w1) {
        const int z = __builtin_clzll(a.w1);
        const uint64_t top = z ? (a.w1 << z) | (a.w0 >> (64 - z)) : a.w1;
        return ldexp((double)top, 64 - z);
    }
    return (double)a.w0;
}

struct quant {
    uint32_t Q;  // < 2^p
    int32_t qe;
};

// RN-even of (a / b) * 2^sh in p bits with gradual underflow at qmin, for 0 <= a < 2^127 and
// 0 < b < 2^127. Returns 0 (result in *y; +0 as Q = 0), 1 when the value rounds beyond the largest
// finite value of a p-bit format with maximum exponent 127, 2 if the quotient estimate could not
// be corrected (unreachable: the estimate is within one unit). Method: the binade of a / b from
// bit lengths and one comparison, then Q = floor(A / B) for A / B < 2^p from an fp64 estimate of
// the quotient, corrected by the exact remainder A - Q B, and rounded by comparing twice the
// remainder with B.
EA_HD inline int rn_quotient(u128 a, u128 b, int64_t sh, int p, int qmin, quant* y) {
    y->Q = 0;
    y->qe = qmin;
    if (a == 0) return 0;
    // a / b lies in (2^-127, 2^127), so shifts beyond +-4096 decide zero and overflow at once
    if (sh < -4096) return 0;
    if (sh > 4096) return 1;
    int k = q_bitlen128(a) - q_bitlen128(b);  // floor(log2(a / b)) is k or k - 1
    if (k >= 0 ? a < (b << k) : (a << -k) < b) --k;
    const int64_t lead = (int64_t)k + sh;  // 2^lead <= (a / b) 2^sh < 2^(lead + 1)
    if (lead < qmin - 1) return 0;         // below half the smallest subnormal: +0
    if (lead > 127) return 1;
    int64_t qe = lead - (p - 1);
    if (qe < qmin) qe = qmin;
    // Q = floor(a 2^s / b), s = sh - qe: A = a 2^s (s > 0, below 2^153) or B = b 2^-s (s < 0,
    // below 2^128); the quotient is below 2^p
    const int s = (int)(sh - qe);
    const w192 A = w192_shifted(a, s > 0 ? s : 0), B = w192_shifted(b, s < 0 ? -s : 0);
    double qd = floor(w192_f64(A) / w192_f64(B));
    qd = qd < 0.0 ? 0.0 : (qd > (double)(1u << p) ? (double)(1u << p) : qd);
    uint32_t Q = (uint32_t)qd;
    w192 QB = w192_mul32(B, Q);
    for (int fix = 0; w192_cmp(QB, A) > 0; ++fix) {
        if (fix == 2) return 2;
        --Q;
        QB = w192_sub(QB, B);
    }
    w192 rem = w192_sub(A, QB);
    for (int fix = 0; w192_cmp(rem, B) >= 0; ++fix) {
        if (fix == 2) return 2;
        ++Q;
        rem = w192_sub(rem, B);
    }
    const int half = w192_cmp(w192_shl(rem, 1), B);  // remainder against half a quantum
    if (half > 0 || (half == 0 && (Q & 1))) ++Q;
    if (Q == (1u << p)) {
        Q >>= 1;
        ++qe;
    }
    if (Q && qe + (31 - __builtin_clz(Q)) > 127) return 1;
    y->Q = Q;
    y->qe = (int32_t)qe;
    return 0;
}

// Sign of (num / den) 2^sh - m 2^e for num < 2^127, 0 < den < 2^127, 0 < m < 2^27: bit lengths
// decide unless the two sides are within a factor of 4, and then both fit 192 bits.
EA_HD inline int cmp_quotient(u128 num, u128 den, int64_t sh, uint32_t m, int64_t e) {
    if (num == 0) return -1;
    const int64_t t = sh - e;  // compare num 2^t with m den
    const int64_t ln = q_bitlen128(num), lm = q_bitlen128(den) + (32 - __builtin_clz(m));
    if (ln - 1 + t >= lm) return 1;   // num 2^t >= 2^lm > m den
    if (ln + t <= lm - 2) return -1;  // num 2^t < 2^(lm - 2) <= m den
    const w192 md = w192_mul32(w192_shifted(den, 0), m);
    if (t >= 0) return w192_cmp(w192_shifted(num, (int)t), md);
    return w192_cmp(w192_shifted(num, 0), w192_shl_any(md, (int)-t));
}

// Bit pattern of (neg ? -1 : 1) Q 2^qe in bf16 (p = 8) or fp32 (p = 24); Q = 0 gives +0.
EA_HD inline uint32_t fmt_bits(uint32_t Q, int qe, bool neg, int fp32) {
    if (Q == 0) return 0;
    const int p = fp32 ? 24 : 8;
    const uint32_t top = 1u << (p - 1);
    // a normal value's biased exponent field is qe + (p - 1) + 127; subnormals sit at qe = qmin
    const uint32_t field = Q >= top ? (uint32_t)(qe + p - 1 + 127) : 0u;
    const uint32_t mag = (field << (p - 1)) + (Q & (top - 1));
    return fp32 ? (mag | (neg ? 0x80000000u : 0u)) : (mag | (neg ? 0x8000u : 0u));
}

// Certified RN of N / Z for N in [Nlo, Nhi] 2^sh and Z in [Zlo, Zhi] (units folded into sh),
// 0 < Zlo <= Zhi, |N| < 2^127. The smallest quotient takes Nlo over the larger Z when Nlo >= 0
// and over the smaller when Nlo < 0; the largest takes Nhi over the smaller Z when Nhi >= 0 and
// over the larger when Nhi < 0. The lower end is rounded; the result is certified when the upper
// end stays inside that result's rounding interval: below its upper midpoint (ties included for
// an even significand) when the result is +0 or positive, at or beyond its lower midpoint in
// magnitude when it is negative (that midpoint a quarter quantum away at the bottom of a binade).
// Returns true with *bits set, false when the interval straddles a rounding boundary or overflows.
EA_HD inline bool certify_quotient(i128 Nlo, i128 Nhi, i128 Zlo, i128 Zhi, int64_t sh, int fp32,
                                        uint32_t* bits) {
    const int p = fp32 ? 24 : 8, qmin = fp32 ? -149 : -133;
    if (Zlo <= 0 || Zhi < Zlo || Nhi < Nlo) return false;
    const bool lo_neg = Nlo < 0;
    quant y;
    if (rn_quotient(lo_neg ? (u128)(-Nlo) : (u128)Nlo, (u128)(lo_neg ? Zlo : Zhi), sh, p, qmin, &y)) return false;
    const bool y_neg = lo_neg && y.Q != 0;
    bool ok;
    if (!y_neg) {
        // the upper end must not pass (2Q + 1) 2^(qe - 1)
        if (Nhi <= 0) {
            ok = true;  // then Nlo <= Nhi <= 0 and y = +0: every value in [L, H] rounds to zero
        } else {
            const int c = cmp_quotient((u128)Nhi, (u128)Zlo, sh, 2 * y.Q + 1, (int64_t)y.qe - 1);
            ok = c < 0 || (c == 0 && !(y.Q & 1));
        }
    } else if (Nhi >= 0) {
        ok = false;  // a negative result with a non-negative upper end
    } else {
        // |upper end| must reach the lower midpoint (2Q - 1) 2^(qe - 1), or (4Q - 1) 2^(qe - 2)
        // when Q opens a binade above the subnormals
        const bool bottom = y.Q == (1u << (p - 1)) && y.qe > qmin;
        const uint32_t m = bottom ? 4 * y.Q - 1 : 2 * y.Q - 1;
        const int64_t e = bottom ? (int64_t)y.qe - 2 : (int64_t)y.qe - 1;
        const int c = cmp_quotient((u128)(-Nhi), (u128)Zhi, sh, m, e);
        ok = c > 0 || (c == 0 && !(y.Q & 1));
    }
    if (ok) *bits = fmt_bits(y.Q, y.qe, y_neg, fp32);
    return ok;
}

}  // namespace ea
