// Device helpers of the certified attention kernels (gfx950). Pure functions on registers.
//
// Tier 1 works in fp64, which CDNA4 executes at the full VALU rate:
//   * a bf16 converts to fp64 exactly; a product of two bf16 is exact in fp64 (16-bit
//     significands); an FMA chain of such products is exact whenever every partial sum fits
//     53 bits above the smallest product's lsb (checked per (row, key) from exponent spreads);
//   * t = RN32(alpha * s) from the exact product split p + e (FMA), with the one double-rounding
//     case (p exactly an fp32 midpoint) resolved by the sign of e;
//   * w = RN24(2^t) by a two-level table with a cubic; relative error below 2^-50.9, so the
//     24-bit rounding is decided unless Y = 2^f * 2^23 lies within 2^-26 of a half-integer;
//   * o = RN(N/Z) from fp64 N, Z with rigorous error bounds: certified when the whole error
//     interval lies strictly between two adjacent rounding midpoints.
// Tier 2 works in 128-bit integers (unsigned __int128 / __int128 compile to 64-bit VALU ops).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ea_quotient.h"
#include "ea_tables.h"

namespace ea {

typedef __int128 i128;
typedef unsigned __int128 u128;

__device__ __forceinline__ double u64_as_f64(uint64_t x) { return __longlong_as_double((long long)x); }
__device__ __forceinline__ uint64_t f64_as_u64(double x) { return (uint64_t)__double_as_longlong(x); }

// bf16 halves of a dword -> fp64 (exact; subnormals need fp32 denormals enabled, which the
// build does with -fno-gpu-flush-denormals-to-zero)
__device__ __forceinline__ double bf16lo_f64(uint32_t w) { return (double)__uint_as_float(w << 16); }
__device__ __forceinline__ double bf16hi_f64(uint32_t w) { return (double)__uint_as_float(w & 0xFFFF0000u); }

// ----------------------------------------------------------------------------------------------
// t = RN32(alpha * s) for an exact fp64 score s and fp32 alpha (as fp64, exact).
// Returns the fp32 bits of t in *t_bits. status: 0 ok, 1 tiny (|t| < 2^-25, so w = 1 exactly),
// 2 overflow (|t| above fp32 max: a domain error).
// ----------------------------------------------------------------------------------------------
__device__ __forceinline__ int logit_rn32(double alpha, double s, uint32_t* t_bits) {
    double p = alpha * s;
    double e = __fma_rn(alpha, s, -p);  // alpha*s = p + e exactly (|p| >= 2^-969 here or tiny)
    double ap = fabs(p);
    if (ap <= 0x1.ffffffcp-26) {  // |alpha s| <= 2^-25 (1 - 2^-29)(1 + 2^-53) < 2^-25
        *t_bits = 0;
        return 1;
    }
    float t0 = (float)p;  // RN-even
    uint32_t b0 = __float_as_uint(t0);
    if ((b0 & 0x7F800000u) == 0x7F800000u) {
        // RN32(p) overflowed. p == 2^128 - 2^103 (the overflow midpoint) with e pulling toward
        // zero would round to the largest finite; everything else overflows.
        if (ap == 0x1.ffffffp127 && (e != 0.0) && ((e < 0.0) == (p > 0.0))) {
            *t_bits = (p > 0.0) ? 0x7F7FFFFFu : 0xFF7FFFFFu;
            return 0;
        }
        return 2;
    }
    double d0 = (double)t0;
    if (d0 != p && e != 0.0) {
        // neighbour on p's side of t0
        bool up_mag = (fabs(p) > fabs(d0));
        uint32_t b1 = up_mag ? b0 + 1 : b0 - 1;
        double d1 = (double)__uint_as_float(b1);
        if (2.0 * p == d0 + d1) {  // p is exactly the midpoint (all terms exact in fp64)
            // x = p + e: the true value lies on e's side of the midpoint
            bool toward_d1 = ((d1 > d0) == (e > 0.0));
            if (toward_d1) b0 = b1;
        }
    }
    *t_bits = b0;
    return 0;
}

// Error-free sum: a + b = s + e exactly (Knuth's TwoSum; any fp64 a, b without overflow).
__device__ __forceinline__ double two_sum(double a, double b, double* e) {
    double s = a + b;
    double bb = s - a;
    *e = (a - (s - bb)) + (b - bb);
    return s;
}

// t = RN32(alpha * x) for a real x known to lie in [s + sig - del, s + sig + del] (fp64 s, sig,
// del >= 0; sig a small correction, |sig| <= 2^-52 |s| or so). Returns 0 and the fp32 bits of t
// when every point of that interval rounds to the same fp32 value, 1 when that value is below
// 2^-25 in magnitude (so w = RN24(2^t) = 1 exactly), 2 when the whole interval overflows fp32
// (a domain error), 3 when undecided.
// alpha*x = p + c with p = RN(alpha s), pe = alpha s - p exact (FMA), c = RN(alpha sig + pe):
// the uncertainty is |c| u + alpha del (+ tiny). RN32 is constant on the open interval between
// the midpoints around t0 = RN32(p); the midpoints are exact in fp64 and p - m is exact there.
__device__ __forceinline__ int logit_cert(double alpha, double s, double sig, double del, uint32_t* t_bits) {
    double p = alpha * s;
    double pe = __fma_rn(alpha, s, -p);
    double c = __fma_rn(alpha, sig, pe);
    double eps = fabs(c) * 0x1p-52 + fabs(alpha) * del * (1.0 + 0x1p-50) + 0x1p-1070;
    double ap = fabs(p);
    if (ap + fabs(c) + eps <= 0x1p-25) {
        *t_bits = 0;
        return 1;
    }
    if (!(ap < 0x1p129)) return (ap >= 0x1p129 && isfinite(p)) ? 2 : 3;
    float t0 = (float)p;  // RN-even
    uint32_t b0 = __float_as_uint(t0);
    if ((b0 & 0x7F800000u) == 0x7F800000u) {
        // |p| rounds past the largest finite: certain overflow unless x could lie below the
        // overflow threshold 2^128 - 2^103
        double thr = 0x1.ffffffp127;
        if (ap - fabs(c) - eps > thr) return 2;
        return 3;
    }
    if (pe == 0.0 && sig == 0.0 && del == 0.0) {  // x = p exactly: RN-even of p (ties included)
        *t_bits = b0;
        return 0;
    }
    // neighbours toward +inf and -inf
    uint32_t mag = b0 & 0x7FFFFFFFu, sg = b0 & 0x80000000u;
    uint32_t up_b = (t0 >= 0.0f) ? ((mag + 1) | sg) : (mag == 0 ? 0x00000001u : ((mag - 1) | sg));
    uint32_t dn_b = (t0 > 0.0f) ? ((mag - 1) | sg) : ((mag + 1) | 0x80000000u);
    if (mag == 0) {
        up_b = 0x00000001u;
        dn_b = 0x80000001u;
    }
    double d0 = (double)t0;
    double m_hi = 0.5 * (d0 + (double)__uint_as_float(up_b));
    double m_lo = 0.5 * (d0 + (double)__uint_as_float(dn_b));
    if (!isfinite(m_hi)) m_hi = 0x1.ffffffp127;  // above the largest finite: the overflow threshold
    if (!isfinite(m_lo)) m_lo = -0x1.ffffffp127;
    double dl = (p - m_lo) + c;  // p - m_lo exact; one rounding
    double dh = (m_hi - p) - c;
    double need = eps + 0x1p-51 * (fabs(dl) + fabs(dh));
    if (dl > need && dh > need) {
        *t_bits = b0;
        return 0;
    }
    return 3;
}

// ----------------------------------------------------------------------------------------------
// w = RN24(2^t) = M * 2^E, M in [2^23, 2^24). fp64 path. Returns 0 certified, 1 undecided
// (|Y - round| too close to a half), 2 out of range (|t| >= 2^30).
// T1/T2 point at the fp64 tables (LDS copies).
// Error analysis (relative, |delta| <= 2^-53 per rounding): T1, T2 entries (2 roundings), their
// product (1), the final FMA (1), the cubic including its truncation (< 2^-67 absolute on a
// value near 1): |y - 2^f| <= 4.01 * 2^-53 * 2^f < 2^-49.9, hence |Y - 2^(f+23)| < 2^-26.9.
// ----------------------------------------------------------------------------------------------
__device__ __forceinline__ int weight_f64(uint32_t t_bits, const double* T1, const double* T2, int32_t* M,
                                          int32_t* E) {
    float tf = __uint_as_float(t_bits);
    uint32_t field = (t_bits >> 23) & 0xFF;
    if (field < 102) {  // |t| < 2^-25: 2^t rounds to 1
        *M = 1 << 23;
        *E = -23;
        return 0;
    }
    if (field >= 127 + 30) return 2;
    double td = (double)tf;
    double n = floor(td);
    double f = td - n;  // exact
    int ni = (int)n;
    if (f == 0.0) {
        *M = 1 << 23;
        *E = ni - 23;
        return 0;
    }
    int i = (int)(f * 65536.0);  // floor, f < 1
    double r = __fma_rn(-(double)i, 0x1p-16, f);  // exact: clears f's top 16 fraction bits
    const double c1 = u64_as_f64(EA_C_BITS[0]), c2 = u64_as_f64(EA_C_BITS[1]), c3 = u64_as_f64(EA_C_BITS[2]);
    double poly = r * __fma_rn(r, __fma_rn(r, c3, c2), c1);
    double a = T1[i >> 8] * T2[i & 255];
    double y = __fma_rn(a, poly, a);
    double Y = y * 8388608.0;  // 2^23, exact
    double fl = floor(Y);
    double fr = Y - fl;  // exact
    if (fabs(fr - 0.5) <= 0x1p-26) return 1;
    int m = (int)fl + (fr > 0.5 ? 1 : 0);
    int e = ni - 23;
    if (m == (1 << 24)) {
        m = 1 << 23;
        ++e;
    }
    *M = m;
    *E = e;
    return 0;
}

// ----------------------------------------------------------------------------------------------
// Certified rounding of a real known to lie in [x - r, x + r] (x, r fp64, r >= 0) to bf16 or
// fp32 (RN-even, gradual underflow, +0 for every zero). Returns true and the bits when every
// point of the interval rounds to the same value.
// ----------------------------------------------------------------------------------------------
// General case: RN of x from its significand, then both neighbouring rounding midpoints at least
// 2r away from |x|.
__device__ __forceinline__ bool certify_round_general(double x, double r, int fp32, uint32_t* bits) {
    const int p = fp32 ? 24 : 8;
    const int qmin = fp32 ? -149 : -133;
    // zero region: |v| <= 2^(qmin-1) rounds to +0 (the boundary is a tie to even zero)
    const double zlim = fp32 ? 0x1p-150 : 0x1p-134;
    double ax = fabs(x);
    if (ax + r <= zlim * (1.0 - 0x1p-40)) {
        *bits = 0;
        return true;
    }
    if (!(ax < 0x1p200) || !(r < 0x1p200)) return false;  // NaN/inf or absurd: not certified
    // RN of x to p bits with the format's subnormal quantum
    uint64_t xb = f64_as_u64(x);
    uint32_t sign = (uint32_t)(xb >> 63);
    int ex = (int)((xb >> 52) & 0x7FF);
    if (ex == 0) return false;  // |x| < 2^-1022: cannot be certified away from zero here
    int k = ex - 1023;  // floor(log2 |x|)
    int qe = k - (p - 1);
    if (qe < qmin) qe = qmin;
    // q = RN(|x| / 2^qe) exactly from the 53-bit significand
    uint64_t mant = (xb & ((1ull << 52) - 1)) | (1ull << 52);  // |x| = mant * 2^(k-52)
    int sh = qe - (k - 52);  // >= 52 - 23 = 29 > 0
    uint64_t q;
    if (sh >= 64) {
        q = 0;  // |x| < 2^(qe-11): rounds to zero; handled by the interval test below
    } else {
        q = mant >> sh;
        uint64_t rem = mant & ((1ull << sh) - 1), half = 1ull << (sh - 1);
        if (rem > half || (rem == half && (q & 1))) ++q;
    }
    // value o = q * 2^qe; neighbours' midpoints
    double o = ldexp((double)q, qe);
    double ulp_up = ldexp(1.0, qe);
    if (q == (1ull << p)) {  // carried into the next binade: o = 2^(qe+p)
        ulp_up = ldexp(1.0, qe + 1);
    }
    double ulp_dn = ldexp(1.0, qe);
    if (q == (1ull << (p - 1)) && qe > qmin) ulp_dn = ldexp(1.0, qe - 1);  // o is a power of two
    if (q == 0) {
        // the interval straddles the zero region boundary
        return false;
    }
    double m_lo = o - 0.5 * ulp_dn, m_hi = o + 0.5 * ulp_up;  // exact
    double dlo = ax - m_lo, dhi = m_hi - ax;  // relative error <= 2^-53 each
    double need = 2.0 * r + 0x1p-1060;
    if (!(dlo > need && dhi > need)) return false;
    // encode |o| in the format
    uint64_t qq = q;
    int e = qe;
    if (qq == (1ull << p)) {
        qq >>= 1;
        ++e;
    }
    if (e + (63 - __clzll(qq)) > 127) return false;  // overflow: never certified
    uint32_t field, frac;
    if (qq < (1ull << (p - 1))) {
        field = 0;
        frac = (uint32_t)qq;
    } else {
        field = (uint32_t)(e - qmin + 1);
        frac = (uint32_t)(qq - (1ull << (p - 1)));
    }
    *bits = (sign << (p - 1 + 8)) | (field << (p - 1)) | frac;
    return true;
}

// Common case in a few integer operations: the interval lies in the format's normal range and
// both of its ends round to the same pattern (rounding is monotone, so every point between does).
// The ends are computed in fp64 on r' = r + |x| 2^-50 + 2^-1070, which covers the rounding of
// the two additions: fl(|x| - r') <= |x| - r and fl(|x| + r') >= |x| + r whenever |x| - r' > 0.
// RN-even to p bits on the fp64 encoding: add 2^(S-1) - 1 plus the kept lsb, drop S = 53 - p
// bits; a carry runs into the exponent field by itself. bf16 and fp32 share fp32's exponent
// range, normal from 2^-126; ends at or above 2^127 are left to the general case.
__device__ __forceinline__ bool certify_round_normal(double x, double r, int fp32, uint32_t* bits) {
    const double ax = fabs(x);
    const double rr = __fma_rn(ax, 0x1p-50, r) + 0x1p-1070;
    const double lo = ax - rr, hi = ax + rr;
    if (!(lo >= 0x1p-126) || !(hi < 0x1p127)) return false;  // also NaN
    const int S = fp32 ? 29 : 45;
    const uint64_t bl = f64_as_u64(lo), bh = f64_as_u64(hi);
    const uint64_t half = (1ull << (S - 1)) - 1;
    const uint64_t ql = (bl + half + ((bl >> S) & 1)) >> S;
    const uint64_t qh = (bh + half + ((bh >> S) & 1)) >> S;
    if (ql != qh) return false;
    // ql = [fp64 exponent field 11 bits][p - 1 fraction bits]: rebias the exponent 1023 -> 127
    const uint32_t sign = (uint32_t)(f64_as_u64(x) >> 63);
    const uint32_t mag = (uint32_t)(ql - ((uint64_t)(1023 - 127) << (52 - S)));
    *bits = (sign << (fp32 ? 31 : 15)) | mag;
    return true;
}

__device__ __forceinline__ bool certify_round(double x, double r, int fp32, uint32_t* bits) {
    if (certify_round_normal(x, r, fp32, bits)) return true;
    return certify_round_general(x, r, fp32, bits);
}

// ----------------------------------------------------------------------------------------------
// 128-bit helpers (tier 2)
// ----------------------------------------------------------------------------------------------
__device__ __forceinline__ int clz64(uint64_t x) { return x ? __clzll(x) : 64; }
__device__ __forceinline__ int bitlen128(u128 x) {
    uint64_t hi = (uint64_t)(x >> 64), lo = (uint64_t)x;
    return hi ? 128 - clz64(hi) : (lo ? 64 - clz64(lo) : 0);
}

// floor / ceil of (a * b) >> 126 for a, b < 2^127
__device__ __forceinline__ u128 mulshr126(u128 a, u128 b, bool up) {
    uint64_t a1 = (uint64_t)(a >> 64), a0 = (uint64_t)a, b1 = (uint64_t)(b >> 64), b0 = (uint64_t)b;
    u128 p00 = (u128)a0 * b0, p01 = (u128)a0 * b1, p10 = (u128)a1 * b0, p11 = (u128)a1 * b1;
    u128 mid = p01 + p10;
    u128 mid_c = mid < p01 ? 1 : 0;
    u128 lo = p00 + (mid << 64);
    u128 lo_c = lo < p00 ? 1 : 0;
    u128 hi = p11 + (mid >> 64) + (mid_c << 64) + lo_c;
    u128 res = (hi << 2) | (lo >> 126);
    if (up && (lo & (((u128)1 << 126) - 1))) ++res;
    return res;
}

__device__ __forceinline__ u128 div_small(u128 a, uint32_t n, bool up) {
    // long division by a 32-bit divisor, 32 bits at a time
    uint64_t r = 0;
    u128 q = 0;
    for (int s = 96; s >= 0; s -= 32) {
        uint64_t cur = (r << 32) | (uint32_t)(a >> s);
        uint64_t qd = cur / n;
        r = cur - qd * n;
        q |= (u128)qd << s;
    }
    if (up && r) ++q;
    return q;
}

// exp(x) * 2^126 enclosure for x in [xl, xh] * 2^-126 with 0 <= x < 2^-8
__device__ __forceinline__ void exp_encl126(u128 xl, u128 xh, u128* lo, u128* hi) {
    const u128 one = (u128)1 << 126;
    u128 s = 0, t = one;
    for (uint32_t n = 1; t != 0 && n < 40; ++n) {
        s += t;
        t = div_small(mulshr126(t, xl, false), n, false);
    }
    *lo = s;
    s = 0;
    t = one;
    for (uint32_t n = 1;; ++n) {
        s += t;
        t = div_small(mulshr126(t, xh, true), n, true);
        if ((t <= 1 && n > 3) || n >= 40) {
            s += 2 * t + 2;
            break;
        }
    }
    *hi = s;
}

// w = RN24(2^t) from a 128-bit fixed-point enclosure (tier 2). 0 certified, 1 undecided,
// 2 out of range (|t| >= 2^62).
__device__ inline int weight_wide(uint32_t t_bits, int32_t* M, int64_t* E) {
    uint32_t field = (t_bits >> 23) & 0xFF;
    if (field < 102) {
        *M = 1 << 23;
        *E = -23;
        return 0;
    }
    if (field >= 127 + 62) return 2;
    int32_t mag = (int32_t)((t_bits & 0x7FFFFF) | 0x800000);
    int32_t tm = (t_bits >> 31) ? -mag : mag;
    int te = (int)field - 150;
    int64_t n;
    uint64_t F;  // f = F * 2^-48
    if (te >= 0) {
        n = (int64_t)tm << te;
        F = 0;
    } else {
        int s = -te;
        n = (int64_t)tm >> s;
        int64_t a = (int64_t)tm - (n << s);
        F = (uint64_t)a << (48 - s);
    }
    if (F == 0) {
        *M = 1 << 23;
        *E = n - 23;
        return 0;
    }
    // 2^f = 2^(j1/256) * 2^(j2/65536) * exp(r ln2), r = R * 2^-48 < 2^-16
    int j1 = (int)(F >> 40), j2 = (int)((F >> 32) & 255);
    uint64_t R = F & 0xFFFFFFFFull;
    const u128 ln2lo = ((u128)EA_LN2W[0] << 64) | EA_LN2W[1];  // floor(ln2 * 2^126)
    const u128 ln2hi = ln2lo + 1;
    u128 xl = mulshr126((u128)R << 78, ln2lo, false);
    u128 xh = mulshr126((u128)R << 78, ln2hi, true);
    u128 el, eh;
    exp_encl126(xl, xh, &el, &eh);
    u128 t1l = ((u128)EA_T1W[2 * j1] << 64) | EA_T1W[2 * j1 + 1], t1h = t1l + 1;
    u128 t2l = ((u128)EA_T2W[2 * j2] << 64) | EA_T2W[2 * j2 + 1], t2h = t2l + 1;
    u128 yl = mulshr126(mulshr126(t1l, t2l, false), el, false);
    u128 yh = mulshr126(mulshr126(t1h, t2h, true), eh, true);
    const int sh = 126 - 23;
    u128 half = (u128)1 << (sh - 1);
    u128 ql = (yl + half) >> sh, qh = (yh + half) >> sh;
    if (ql != qh) return 1;
    int64_t e = n - 23;
    if (ql == ((u128)1 << 24)) {
        ql >>= 1;
        ++e;
    }
    *M = (int32_t)ql;
    *E = e;
    return 0;
}

// (W >> s) mod 2^64 for the 192-bit W = (w2 : w1 : w0) and s >= 0
__device__ __forceinline__ uint64_t shr192(uint64_t w2, uint64_t w1, uint64_t w0, int s) {
    if (s >= 192) return 0;
    if (s >= 128) return w2 >> (s - 128);
    if (s >= 64) return s == 64 ? w1 : (w1 >> (s - 64)) | (w2 << (128 - s));
    return s == 0 ? w0 : (w0 >> s) | (w1 << (64 - s));
}
// any of bits [0, m) of W set, m >= 0
__device__ __forceinline__ bool low_bits192(uint64_t w2, uint64_t w1, uint64_t w0, int m) {
    if (m >= 192) return (w0 | w1 | w2) != 0;
    if (m >= 128) return (w0 | w1) != 0 || (m > 128 && (w2 & ((1ull << (m - 128)) - 1)) != 0);
    if (m >= 64) return w0 != 0 || (m > 64 && (w1 & ((1ull << (m - 64)) - 1)) != 0);
    return m > 0 && (w0 & ((1ull << m) - 1)) != 0;
}

// RN32 of (am * X) * 2^E with X a signed 128-bit integer and |am| < 2^24: the exact logit.
// status 0 ok, 2 overflow. Zero gives bits 0. The 152-bit product stays in three 64-bit words;
// the kept bits, the rounding bit and the sticky bit come from word shifts (no bit loops, no
// indexed arrays).
__device__ inline int rn32_prod(int32_t am, i128 X, int E, uint32_t* bits) {
    if (X == 0 || am == 0) {
        *bits = 0;
        return 0;
    }
    const int sign = ((X < 0) != (am < 0)) ? -1 : 1;
    const u128 ax = X < 0 ? (u128)(-X) : (u128)X;
    const uint64_t aa = (uint64_t)(am < 0 ? -(int64_t)am : am);
    const u128 lo = (u128)(uint64_t)ax * aa;
    const u128 hi = (u128)(uint64_t)(ax >> 64) * aa + (lo >> 64);
    const uint64_t w0 = (uint64_t)lo, w1 = (uint64_t)hi, w2 = (uint64_t)(hi >> 64);
    const int bl = w2 ? 192 - __clzll(w2) : (w1 ? 128 - __clzll(w1) : 64 - __clzll(w0));
    const long k = (long)bl - 1 + E;  // floor(log2 |am X 2^E|)
    long qe = k - 23;
    if (qe < -149) qe = -149;
    const long lo_bit = qe - E;  // position in W of the result's last kept bit
    uint64_t q;
    bool rb = false, st = false;
    if (lo_bit <= 0) {
        // every bit kept: W < 2^24 and -lo_bit < 24 (qe = k - 23, or the clamp with k < -127)
        q = w0 << (-lo_bit);
    } else {
        q = shr192(w2, w1, w0, (int)lo_bit);
        rb = (shr192(w2, w1, w0, (int)lo_bit - 1) & 1) != 0;
        st = low_bits192(w2, w1, w0, (int)lo_bit - 1);
    }
    if (rb && (st || (q & 1))) ++q;
    if (q == (1ull << 24)) {
        q >>= 1;
        ++qe;
    }
    if (q && qe + (63 - __clzll(q)) > 127) return 2;
    *bits = fmt_bits((uint32_t)q, (int)qe, sign < 0, 1);
    return 0;
}

}  // namespace ea
