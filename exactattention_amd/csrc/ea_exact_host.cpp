// Host exact tier: one attention row with exact integer arithmetic (see ea_exact.h).
//
//   scores   s = sum_i q_i k_i as one multiword integer at the smallest product exponent (bf16
//            products span at most 2^16 x 2^506: ten 64-bit words hold any sum of 128 of them)
//   logit    t = RN32(alpha s) by exact division-free rounding of am |S| 2^(ae + es)
//   weight   w = RN24(2^t): integer t gives a power of two; otherwise 2^f (f = t - floor t) is
//            irrational, and integer enclosures of ln 2 and of the exponential series at W bits,
//            W doubling until both ends round alike, decide it (Ziv's strategy)
//   sums     Z = sum w_j and N_c = sum w_j v_jc in windows of W bits below their largest term:
//            terms below the window are floored and counted, so the true sums lie in
//            [sum, sum + count] units; RN(N_c / Z) is taken when both ends of the interval round
//            alike, else W doubles. Once W covers every term the sums are exact and the rounding
//            is always decided, so the loop ends for every finite input.
// The definition is the reference's (docs/SPEC.md:8-80, src/exactattn/reference.py:47-143);
// the multiword routines, the ln 2 series (2 atanh(1/3)) and the window scheme are this
// library's own.
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <new>
#include <vector>

#include "ea_exact.h"

namespace eax {
namespace {

typedef unsigned __int128 u128;
typedef __int128 i128;

// ------------------------------------------------------------------------------------------------
// Unsigned multiword integers: little-endian 64-bit words, no leading zero words.
// ------------------------------------------------------------------------------------------------
struct Big {
    std::vector<uint64_t> w;
    bool zero() const { return w.empty(); }
    void trim() {
        while (!w.empty() && w.back() == 0) w.pop_back();
    }
};

Big big_u64(uint64_t x) {
    Big r;
    if (x) r.w.push_back(x);
    return r;
}

Big big_u128(u128 x) {
    Big r;
    r.w.push_back((uint64_t)x);
    r.w.push_back((uint64_t)(x >> 64));
    r.trim();
    return r;
}

int64_t bitlen(const Big& a) {
    return a.w.empty() ? 0 : 64 * (int64_t)(a.w.size() - 1) + (64 - __builtin_clzll(a.w.back()));
}

int cmp(const Big& a, const Big& b) {
    if (a.w.size() != b.w.size()) return a.w.size() < b.w.size() ? -1 : 1;
    for (size_t i = a.w.size(); i-- > 0;)
        if (a.w[i] != b.w[i]) return a.w[i] < b.w[i] ? -1 : 1;
    return 0;
}

Big shl(const Big& a, int64_t s) {
    if (a.zero() || s == 0) return a;
    Big r;
    const size_t ws = (size_t)(s / 64);
    const int bs = (int)(s % 64);
    r.w.assign(ws + a.w.size() + 1, 0);
    for (size_t i = 0; i < a.w.size(); ++i) {
        r.w[ws + i] |= a.w[i] << bs;
        if (bs) r.w[ws + i + 1] |= a.w[i] >> (64 - bs);
    }
    r.trim();
    return r;
}

// floor(a / 2^s)
Big shr(const Big& a, int64_t s) {
    const size_t ws = (size_t)(s / 64);
    const int bs = (int)(s % 64);
    if (ws >= a.w.size()) return Big();
    Big r;
    r.w.assign(a.w.size() - ws, 0);
    for (size_t i = 0; i < r.w.size(); ++i) {
        r.w[i] = a.w[ws + i] >> bs;
        if (bs && ws + i + 1 < a.w.size()) r.w[i] |= a.w[ws + i + 1] << (64 - bs);
    }
    r.trim();
    return r;
}

// true when a has a one bit below position s
bool low_bits(const Big& a, int64_t s) {
    const size_t ws = (size_t)(s / 64);
    const int bs = (int)(s % 64);
    for (size_t i = 0; i < ws && i < a.w.size(); ++i)
        if (a.w[i]) return true;
    return bs && ws < a.w.size() && (a.w[ws] & ((1ull << bs) - 1));
}

void add_to(Big& a, const Big& b) {
    if (a.w.size() < b.w.size()) a.w.resize(b.w.size(), 0);
    uint64_t c = 0;
    for (size_t i = 0; i < a.w.size(); ++i) {
        const u128 s = (u128)a.w[i] + (i < b.w.size() ? b.w[i] : 0) + c;
        a.w[i] = (uint64_t)s;
        c = (uint64_t)(s >> 64);
        if (!c && i >= b.w.size()) break;
    }
    if (c) a.w.push_back(c);
}

void add_small(Big& a, uint64_t x) { add_to(a, big_u64(x)); }

// a -= b, a >= b
void sub_from(Big& a, const Big& b) {
    uint64_t br = 0;
    for (size_t i = 0; i < a.w.size(); ++i) {
        const uint64_t bi = i < b.w.size() ? b.w[i] : 0;
        const u128 s = (u128)a.w[i] - bi - br;
        a.w[i] = (uint64_t)s;
        br = (uint64_t)(s >> 64) ? 1 : 0;
        if (!br && i >= b.w.size()) break;
    }
    a.trim();
}

Big mul(const Big& a, const Big& b) {
    Big r;
    if (a.zero() || b.zero()) return r;
    r.w.assign(a.w.size() + b.w.size(), 0);
    for (size_t i = 0; i < a.w.size(); ++i) {
        uint64_t c = 0;
        for (size_t j = 0; j < b.w.size(); ++j) {
            const u128 t = (u128)a.w[i] * b.w[j] + r.w[i + j] + c;
            r.w[i + j] = (uint64_t)t;
            c = (uint64_t)(t >> 64);
        }
        r.w[i + b.w.size()] = c;
    }
    r.trim();
    return r;
}

// a = floor(a / d), returns a mod d (d > 0)
uint64_t divmod_small(Big& a, uint64_t d) {
    u128 r = 0;
    for (size_t i = a.w.size(); i-- > 0;) {
        const u128 cur = (r << 64) | a.w[i];
        a.w[i] = (uint64_t)(cur / d);
        r = cur % d;
    }
    a.trim();
    return (uint64_t)r;
}

// ceil(a / d)
Big div_ceil_small(const Big& a, uint64_t d) {
    Big q = a;
    if (divmod_small(q, d)) add_small(q, 1);
    return q;
}

// ------------------------------------------------------------------------------------------------
// Rounding: RN-even of (a / b) * 2^E into p bits with minimum quantum qmin (gradual underflow).
// The result is Q * 2^qe with Q < 2^p (Q < 2^(p-1) only at qe = qmin); Q = 0 when the value
// rounds to zero.
// ------------------------------------------------------------------------------------------------
struct Rounded {
    uint32_t Q;
    int64_t qe;
};

Rounded round_ratio(const Big& a, const Big& b, int64_t E, int p, int qmin) {
    Rounded r{0, qmin};
    if (a.zero()) return r;
    const int64_t L = bitlen(a) - bitlen(b);
    // 2^(L - 1) < a / b < 2^(L + 1). Below half the smallest quantum the value rounds to zero;
    // far above every format's range it overflows. Both are decided here, before any shift by
    // E, so that no operand ever grows with |E| (E can be of order 2^40 for a row whose weights
    // lie that far apart).
    if (L + 1 + E <= (int64_t)qmin - 1) return r;
    if (L - 1 + E > 4096) {
        r.Q = 1u << (p - 1);
        r.qe = L - 1 + E - (p - 1);
        return r;
    }
    const bool ge = L >= 0 ? cmp(a, shl(b, L)) >= 0 : cmp(shl(a, -L), b) >= 0;
    const int64_t lead = ge ? L : L - 1;  // 2^lead <= a / b < 2^(lead + 1)
    int64_t qe = lead + E - (p - 1);
    if (qe < qmin) qe = qmin;
    const int64_t s = E - qe;  // value / 2^qe = a 2^s / b < 2^p
    Big n = s >= 0 ? shl(a, s) : a;
    const Big d = s >= 0 ? b : shl(b, -s);
    uint64_t Q = 0;
    for (int i = p; i >= 0; --i) {
        const Big di = shl(d, i);
        if (cmp(n, di) >= 0) {
            sub_from(n, di);
            Q |= 1ull << i;
        }
    }
    const int c = cmp(shl(n, 1), d);  // the remainder against half a quantum
    if (c > 0 || (c == 0 && (Q & 1))) ++Q;
    if (Q == (1ull << p)) {
        Q >>= 1;
        ++qe;
    }
    r.Q = (uint32_t)Q;
    r.qe = Q ? qe : qmin;
    return r;
}

// bit pattern of sign * Q * 2^qe (a value round_ratio produced) in bf16 or fp32; +0 for Q = 0
uint32_t encode(const Rounded& r, bool neg, int fp32) {
    if (r.Q == 0) return 0;
    const int p = fp32 ? 24 : 8;
    const int64_t bias = fp32 ? 150 : 134;  // field of a normal value Q 2^qe with Q >= 2^(p-1)
    const uint32_t field = r.Q >= (1u << (p - 1)) ? (uint32_t)(r.qe + bias) : 0u;
    const uint32_t frac = r.Q & ((1u << (p - 1)) - 1);
    const uint32_t mag = (field << (p - 1)) | frac;
    return fp32 ? (mag | (neg ? 0x80000000u : 0u)) : (mag | (neg ? 0x8000u : 0u));
}

bool overflows(const Rounded& r, int fp32) {
    // largest finite: field 254 (bf16 qe = 120, fp32 qe = 104) with a full significand
    return r.Q && r.qe > (fp32 ? 104 : 120);
}

// ------------------------------------------------------------------------------------------------
// ln 2 and 2^f enclosures
// ------------------------------------------------------------------------------------------------

// lo <= ln(2) 2^W <= hi from ln 2 = 2 atanh(1/3) = sum_k 2 / ((2k + 1) 3^(2k + 1)). The powers of
// three are divided out one factor 9 at a time (nested floors and ceilings of integer division
// equal the single ones); the tail after the last term is below 9/8 of a value under 1.
void ln2_enclosure(int W, Big& lo, Big& hi) {
    static std::mutex mu;
    static std::vector<std::pair<int, std::pair<Big, Big>>> cache;
    {
        std::lock_guard<std::mutex> g(mu);
        for (auto& c : cache)
            if (c.first == W) {
                lo = c.second.first;
                hi = c.second.second;
                return;
            }
    }
    Big P = shl(big_u64(2), W), C = P;
    divmod_small(P, 3);
    C = div_ceil_small(C, 3);
    lo = Big();
    hi = Big();
    for (uint64_t k = 0; !P.zero(); ++k) {
        Big t = P;
        divmod_small(t, 2 * k + 1);
        add_to(lo, t);
        add_to(hi, div_ceil_small(C, 2 * k + 1));
        divmod_small(P, 9);
        C = div_ceil_small(C, 9);
    }
    add_small(hi, 2);
    std::lock_guard<std::mutex> g(mu);
    cache.push_back({W, {lo, hi}});
}

// exp(x) 2^W enclosed for x in [xlo, xhi] 2^-W, 0 <= x < 1: the Taylor terms of xlo floored
// (every term is positive, so the truncated sum is a lower bound), of xhi ceiled, plus twice the
// first omitted term for the tail (x / (n + 1) <= 1/2 from n = 1 on) and one unit of slack.
void exp_enclosure(const Big& xlo, const Big& xhi, int W, Big& ylo, Big& yhi) {
    const Big one = shl(big_u64(1), W);
    ylo = Big();
    Big t = one;
    for (uint64_t n = 1; !t.zero(); ++n) {
        add_to(ylo, t);
        t = shr(mul(t, xlo), W);
        divmod_small(t, n);
    }
    yhi = Big();
    t = one;
    for (uint64_t n = 1;; ++n) {
        add_to(yhi, t);
        Big u = mul(t, xhi);
        const bool frac = low_bits(u, W);
        u = shr(u, W);
        if (frac) add_small(u, 1);
        t = div_ceil_small(u, n);
        if (n > 3 && cmp(t, big_u64(1)) <= 0) {
            add_to(yhi, shl(t, 1));
            add_small(yhi, 1);
            break;
        }
    }
}

// w = RN24(2^t) = M 2^E for t = tm 2^te (an fp32 value). Returns false only if the enclosure
// failed to converge by 2^16 bits (never observed: 2^f is irrational for non-integer f).
bool weight_exact(int32_t tm, int32_t te, uint32_t* M, i128* E) {
    if (tm == 0) {
        *M = 1u << 23;
        *E = -23;
        return true;
    }
    if (te >= 0) {
        *M = 1u << 23;
        *E = ((i128)tm << te) - 23;
        return true;
    }
    const int k = -te;
    // t = n + a 2^-k with n = floor(t), 0 <= a < 2^k
    int64_t n;
    Big a;
    if (k < 32) {
        n = (int64_t)tm >> k;  // arithmetic shift: floor
        a = big_u64((uint64_t)((int64_t)tm - n * ((int64_t)1 << k)));
    } else if (tm > 0) {
        n = 0;
        a = big_u64((uint64_t)tm);
    } else {
        n = -1;
        a = shl(big_u64(1), k);
        sub_from(a, big_u64((uint64_t)(-(int64_t)tm)));
    }
    if (a.zero()) {
        *M = 1u << 23;
        *E = (i128)n - 23;
        return true;
    }
    for (int W = 96; W <= (1 << 16); W *= 2) {
        Big Llo, Lhi;
        ln2_enclosure(W, Llo, Lhi);
        const Big xlo = shr(mul(a, Llo), k);
        Big u = mul(a, Lhi);
        const bool frac = low_bits(u, k);
        Big xhi = shr(u, k);
        if (frac) add_small(xhi, 1);
        Big ylo, yhi;
        exp_enclosure(xlo, xhi, W, ylo, yhi);
        // M = round(2^f 2^23): the value y 2^(23 - W) rounded half up (2^f is never a midpoint)
        const int sh = W - 23;
        Big qlo = ylo, qhi = yhi;
        add_to(qlo, shl(big_u64(1), sh - 1));
        add_to(qhi, shl(big_u64(1), sh - 1));
        qlo = shr(qlo, sh);
        qhi = shr(qhi, sh);
        if (cmp(qlo, qhi) == 0) {
            uint64_t q = qlo.zero() ? 0 : qlo.w[0];
            i128 e = (i128)n - 23;
            if (q == (1ull << 24)) {
                q >>= 1;
                e += 1;
            }
            *M = (uint32_t)q;
            *E = e;
            return true;
        }
    }
    return false;
}

// ------------------------------------------------------------------------------------------------
// bf16 decode: value m 2^e, |m| < 256 (bit 7 set for normal values); false for NaN/inf
// ------------------------------------------------------------------------------------------------
inline bool dec_bf16(uint16_t x, int* m, int* e) {
    const int f = (x >> 7) & 0xFF;
    if (f == 0xFF) return false;
    const int mm = (x & 0x7F) | (f ? 0x80 : 0);
    *m = (x & 0x8000) ? -mm : mm;
    *e = (f ? f : 1) - 134;
    return true;
}

// Windowed sum of signed terms x_j 2^e_j (|x_j| < 2^32): terms floored to units 2^base, the true
// sum in [pos - neg, pos - neg + lost] units.
struct WSum {
    std::vector<uint64_t> pos, neg;
    uint64_t lost = 0;
    void init(size_t words) {
        pos.assign(words, 0);
        neg.assign(words, 0);
        lost = 0;
    }
    static void add_at(std::vector<uint64_t>& a, uint64_t x, int64_t s) {
        size_t i = (size_t)(s / 64);
        const int bs = (int)(s % 64);
        u128 v = (u128)x << bs;
        while (v && i < a.size()) {
            const u128 t = (u128)a[i] + (uint64_t)v;
            a[i] = (uint64_t)t;
            v = (v >> 64) + (t >> 64);
            ++i;
        }
    }
    void add(uint64_t x, bool negative, i128 e, i128 base) {
        if (!x) return;
        const i128 s = e - base;
        uint64_t tr;
        bool ls;
        if (s >= 0) {
            tr = x;
            ls = false;
            add_at(negative ? neg : pos, tr, (int64_t)s);
            return;
        }
        if (s <= -64) {
            tr = 0;
            ls = true;
        } else {
            const int sh = (int)(-s);
            tr = x >> sh;
            ls = (tr << sh) != x;
        }
        lost += ls ? 1 : 0;
        if (negative) tr += ls ? 1 : 0;  // floor(-x) = -ceil(x)
        if (tr) add_at(negative ? neg : pos, tr, 0);
    }
};

Big from_words(const std::vector<uint64_t>& w) {
    Big r;
    r.w = w;
    r.trim();
    return r;
}

// signed multiword value: magnitude and sign
struct SBig {
    Big m;
    bool neg = false;
};

SBig signed_diff(const Big& p, const Big& n) {
    SBig r;
    if (cmp(p, n) >= 0) {
        r.m = p;
        sub_from(r.m, n);
    } else {
        r.m = n;
        sub_from(r.m, p);
        r.neg = true;
    }
    if (r.m.zero()) r.neg = false;
    return r;
}

SBig add_u64(const SBig& a, uint64_t x) {
    SBig r = a;
    if (!x) return r;
    if (!r.neg) {
        add_small(r.m, x);
        return r;
    }
    const Big bx = big_u64(x);
    if (cmp(r.m, bx) >= 0) {
        sub_from(r.m, bx);
        if (r.m.zero()) r.neg = false;
    } else {
        Big t = bx;
        sub_from(t, r.m);
        r.m = t;
        r.neg = false;
    }
    return r;
}

// bits of RN(num / den * 2^E) for a signed numerator and den > 0
uint32_t round_signed(const SBig& num, const Big& den, i128 E, int fp32) {
    // |num / den| 2^E < 2^(bitlen(num) + 1 - bitlen(den) + E): below half the smallest subnormal
    // it rounds to +0 (round_ratio makes the same test; this one also keeps E within int64).
    // Numerators never sit far above their denominators (E <= 160).
    if (num.m.zero()) return 0;
    const int qmin = fp32 ? -149 : -133;
    if ((i128)bitlen(num.m) + 1 - bitlen(den) + E <= qmin - 1) return 0;
    const Rounded r = round_ratio(num.m, den, (int64_t)E, fp32 ? 24 : 8, qmin);
    return encode(r, num.neg, fp32);
}

const i128 SPREAD_LIMIT = (i128)1 << 20;

}  // namespace

namespace {

int exact_row_body(const uint16_t* q, int d, const uint16_t* K, const uint16_t* V, int64_t n, int dv,
                   uint32_t alpha_bits, int fp32, void* out, const KeyTrace* tr) {
    std::vector<int> qm(d), qe(d);
    for (int i = 0; i < d; ++i)
        if (!dec_bf16(q[i], &qm[i], &qe[i])) return EAX_DOMAIN;
    for (int64_t j = 0; j < n; ++j) {
        int m, e;
        for (int i = 0; i < d; ++i)
            if (!dec_bf16(K[j * d + i], &m, &e)) return EAX_DOMAIN;
        for (int c = 0; c < dv; ++c)
            if (!dec_bf16(V[j * dv + c], &m, &e)) return EAX_DOMAIN;
    }
    const uint32_t ab = alpha_bits;
    const int af = (ab >> 23) & 0xFF;
    if (af == 0xFF) return EAX_DOMAIN;
    const int32_t am_abs = (int32_t)((ab & 0x7FFFFF) | (af ? 0x800000 : 0));
    const bool a_neg = (ab >> 31) != 0;
    const int32_t ae = (af ? af : 1) - 150;

    // ---- scores and logits
    std::vector<int32_t> tmv((size_t)n), tev((size_t)n);
    std::vector<uint32_t> tbv((size_t)n);
    for (int64_t j = 0; j < n; ++j) {
        // exact score at the fixed exponent -266 (the smallest product exponent of two bf16s):
        // every product is |m| < 2^16 at an offset below 2^9
        Big P, N;
        std::vector<uint64_t> pw(10, 0), nw(10, 0);
        for (int i = 0; i < d; ++i) {
            int km, ke;
            dec_bf16(K[j * d + i], &km, &ke);
            const int pm = qm[i] * km;
            if (!pm) continue;
            const int64_t s = (int64_t)qe[i] + ke + 266;
            WSum::add_at(pm > 0 ? pw : nw, (uint64_t)(pm > 0 ? pm : -pm), s);
        }
        const SBig S = signed_diff(from_words(pw), from_words(nw));
        int32_t tm = 0, te = 0;
        uint32_t tbits = 0;
        if (!S.m.zero() && am_abs) {
            const Big prod = mul(S.m, big_u64((uint64_t)am_abs));
            const Rounded r = round_ratio(prod, big_u64(1), (int64_t)ae - 266, 24, -149);
            if (overflows(r, 1)) return EAX_DOMAIN;  // |alpha s| rounds above the fp32 range
            const bool tneg = S.neg != a_neg;
            tm = tneg ? -(int32_t)r.Q : (int32_t)r.Q;
            te = (int32_t)r.qe;
            tbits = encode(r, tneg, 1);
        }
        tmv[(size_t)j] = tm;
        tev[(size_t)j] = te;
        tbv[(size_t)j] = tbits;
    }
    // Logits of magnitude 2^100 or more (fp32 field >= 227): weight exponents t - 23 need more than
    // 128 bits near 2^128. Distinct such logits differ by at least 2^76, beyond the exponent-spread
    // limit (the reference refuses those rows too, reference.py:109-110); equal ones give equal
    // weights, whose common factor 2^t cancels in N / Z, so every weight is taken as 1.
    bool huge = false, same = true;
    for (int64_t j = 0; j < n; ++j) {
        huge |= ((tbv[(size_t)j] >> 23) & 0xFF) >= 227;
        same &= tbv[(size_t)j] == tbv[0];
    }
    if (huge && !same) return EAX_REFUSED;

    // ---- weights
    std::vector<uint32_t> wM((size_t)n);
    std::vector<i128> wE((size_t)n);
    const i128 lim = (i128)1 << 62;  // trace exponents are clamped to +-2^62
    for (int64_t j = 0; j < n; ++j) {
        uint32_t M = 1u << 23;
        i128 E = -23;
        int64_t we_trace;
        if (huge) {
            we_trace = (tmv[(size_t)j] < 0) ? -lim : lim;  // t - 23 for |t| >= 2^100
        } else {
            if (!weight_exact(tmv[(size_t)j], tev[(size_t)j], &M, &E)) return EAX_REFUSED;
            we_trace = (int64_t)(E > lim ? lim : (E < -lim ? -lim : E));
        }
        wM[(size_t)j] = M;
        wE[(size_t)j] = E;
        if (tr) {
            if (tr->t_bits) tr->t_bits[j] = tbv[(size_t)j];
            if (tr->wm) tr->wm[j] = (int32_t)M;
            if (tr->we) tr->we[j] = we_trace;
        }
    }
    uint16_t* o16 = (uint16_t*)out;
    uint32_t* o32 = (uint32_t*)out;
    if (n == 0) {
        for (int c = 0; c < dv; ++c) {
            if (fp32) o32[c] = 0;
            else o16[c] = 0;
        }
        return EAX_OK;
    }

    // ---- Z and N_c in windows of W bits below their largest terms
    i128 emax = wE[0], emin = wE[0];
    for (int64_t j = 1; j < n; ++j) {
        emax = std::max(emax, wE[(size_t)j]);
        emin = std::min(emin, wE[(size_t)j]);
    }
    const i128 ztop = emax + 24;  // every weight is below 2^ztop
    const i128 zfull = ztop - emin;
    // per channel: top of the largest term and the lowest term exponent
    std::vector<i128> ntop(dv), nlow(dv);
    std::vector<int> nonzero(dv, 0);
    for (int c = 0; c < dv; ++c) {
        i128 top = 0, low = 0;
        bool any = false;
        for (int64_t j = 0; j < n; ++j) {
            int m, e;
            dec_bf16(V[j * dv + c], &m, &e);
            if (!m) continue;
            const uint64_t x = (uint64_t)wM[(size_t)j] * (uint64_t)(m < 0 ? -m : m);
            const i128 ex = wE[(size_t)j] + e;
            const i128 t = ex + (64 - __builtin_clzll(x));
            if (!any || t > top) top = t;
            if (!any || ex < low) low = ex;
            any = true;
        }
        ntop[c] = top;
        nlow[c] = low;
        nonzero[c] = any;
    }
    std::vector<int> done(dv, 0);
    std::vector<uint32_t> bits(dv, 0);
    for (int c = 0; c < dv; ++c)
        if (!nonzero[c]) done[c] = 1;  // N_c = 0 exactly: +0
    for (int64_t W = 160;; W *= 2) {
        // Z at this width (exact once W covers every weight)
        const i128 zbase = ztop - W;
        WSum zs;
        zs.init((size_t)(W / 64 + 2));
        for (int64_t j = 0; j < n; ++j) zs.add(wM[(size_t)j], false, wE[(size_t)j], zbase);
        const Big zlo = from_words(zs.pos);
        Big zhi = zlo;
        add_small(zhi, zs.lost);
        bool all = true;
        bool any_capped = false;
        for (int c = 0; c < dv; ++c) {
            if (done[c]) continue;
            const i128 nbase = ntop[c] - W;
            WSum ns;
            ns.init((size_t)(W / 64 + 2));
            for (int64_t j = 0; j < n; ++j) {
                int m, e;
                dec_bf16(V[j * dv + c], &m, &e);
                if (!m) continue;
                ns.add((uint64_t)wM[(size_t)j] * (uint64_t)(m < 0 ? -m : m), m < 0, wE[(size_t)j] + e, nbase);
            }
            const SBig nlo = signed_diff(from_words(ns.pos), from_words(ns.neg));
            const SBig nhi = add_u64(nlo, ns.lost);
            const i128 E = nbase - zbase;
            // sign-aware ends of [nlo, nhi] / [zlo, zhi]
            uint32_t blo, bhi;
            if (!nlo.neg) {
                blo = round_signed(nlo, zhi, E, fp32);
                bhi = round_signed(nhi, zlo, E, fp32);
            } else if (nhi.neg || nhi.m.zero()) {
                blo = round_signed(nlo, zlo, E, fp32);
                bhi = round_signed(nhi, zhi, E, fp32);
            } else {
                blo = round_signed(nlo, zlo, E, fp32);
                bhi = round_signed(nhi, zlo, E, fp32);
            }
            if (blo == bhi) {
                bits[c] = blo;
                done[c] = 1;
                continue;
            }
            all = false;
            const i128 full = std::max(zfull, ntop[c] - nlow[c]);
            if (W >= full && zs.lost == 0 && ns.lost == 0) {
                // cannot happen: exact sums round to one pattern
                return EAX_REFUSED;
            }
            if (full > SPREAD_LIMIT + 64) any_capped = true;
        }
        if (all) break;
        if (any_capped && W > SPREAD_LIMIT) return EAX_REFUSED;
    }
    for (int c = 0; c < dv; ++c) {
        if (fp32) o32[c] = bits[c];
        else o16[c] = (uint16_t)bits[c];
    }
    return EAX_OK;
}

}  // namespace

int exact_row(const uint16_t* q, int d, const uint16_t* K, const uint16_t* V, int64_t n, int dv, uint32_t alpha_bits,
              int fp32, void* out, const KeyTrace* tr) noexcept {
    try {
        return exact_row_body(q, d, K, V, n, dv, alpha_bits, fp32, out, tr);
    } catch (const std::bad_alloc&) {
        return EAX_NOMEM;
    } catch (...) {
        return EAX_NOMEM;
    }
}

uint32_t round_ratio_bits(uint64_t a_hi, uint64_t a_lo, uint64_t b_hi, uint64_t b_lo, int64_t E, int neg, int fp32,
                          int* overflow) noexcept {
    *overflow = 0;
    try {
        const Big a = big_u128(((u128)a_hi << 64) | a_lo), b = big_u128(((u128)b_hi << 64) | b_lo);
        if (b.zero() || a.zero()) return 0;
        const Rounded r = round_ratio(a, b, E, fp32 ? 24 : 8, fp32 ? -149 : -133);
        if (overflows(r, fp32)) {
            *overflow = 1;
            return 0;
        }
        return encode(r, neg != 0, fp32);
    } catch (...) {  // operands are at most 128 bits plus p: only an exhausted heap gets here
        *overflow = 1;
        return 0;
    }
}

}  // namespace eax
