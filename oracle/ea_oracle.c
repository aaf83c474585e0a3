/*
 * CPU oracle, part 2: the reference's certified CPU algorithm restated in C.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg load this library, and only as the checker. The product never links it.
 *
 * Restates csrc/exact_attention_cpu.cpp (reference checkout) function by function:
 *   round_ratio        exact RN of (a/b)*2^E                       (:111-153)
 *   decode_bf16/fp32                                               (:169-199)
 *   score + logit      the reference windows an int64 sum (:215-255); here the score is
 *                      exact (redundant 32-bit limbs, 640 bits), so t = RN32(alpha*s) is exact
 *   weight             the reference uses libm exp2 with a margin (:260-291); here an integer
 *                      interval enclosure of 2^f at 2^-126 decides RN24 (own method)
 *   tile_partial       per-tile Z and per-channel N with per-term anchor (:361-401)
 *   merge_into         order-free merge with counted truncation (:403-441)
 *   finalize           certified final rounding of both interval ends (:450-490)
 *   run_rows           splits x tiles, seeded merge order, flags 0/1/2 (:511-574)
 *   ea_attention_cpu   same C ABI and argument meaning (:585-628)
 * plus oracle_attention_geom(), which evaluates the same rows from the serving geometry the GPU
 * library takes (paged KV, GQA segments, prefix lengths, tree masks) without building a CSR.
 *
 * Rows whose result this code cannot certify are flagged 1; the Python exact oracle
 * (oracle/exact.py) recomputes those. Flag 2 = non-finite input or fp32 logit overflow.
 * The seeded merge order uses splitmix64 + Fisher-Yates (the reference uses std::shuffle,
 * whose sequence is implementation-defined); certified bits cannot depend on it.
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef __int128 i128;
typedef unsigned __int128 u128;
typedef int64_t i64;
typedef uint64_t u64;

/* ------------------------------------------------------------------------------------------
 * Small unsigned multiword integers, 32-bit limbs, little-endian.
 * ---------------------------------------------------------------------------------------- */
#define MW 24 /* 768 bits */
typedef struct { uint32_t w[MW]; } mw;

static void mw_zero(mw* a) { memset(a, 0, sizeof(*a)); }
static void mw_from_u128(mw* a, u128 x) {
    mw_zero(a);
    for (int i = 0; i < 4; ++i) a->w[i] = (uint32_t)(x >> (32 * i));
}
static int mw_bitlen(const mw* a) {
    for (int i = MW - 1; i >= 0; --i)
        if (a->w[i]) return 32 * i + (32 - __builtin_clz(a->w[i]));
    return 0;
}
static int mw_bit(const mw* a, int i) { return (i < 0 || i >= 32 * MW) ? 0 : (a->w[i >> 5] >> (i & 31)) & 1; }
static int mw_any_below(const mw* a, int i) { /* any set bit at positions < i */
    if (i <= 0) return 0;
    if (i >= 32 * MW) i = 32 * MW;
    int L = i >> 5;
    for (int j = 0; j < L; ++j)
        if (a->w[j]) return 1;
    if (i & 31) return (a->w[L] & ((1u << (i & 31)) - 1)) != 0;
    return 0;
}
static void mw_shl(mw* r, const mw* a, int s) {
    mw t;
    mw_zero(&t);
    int L = s >> 5, b = s & 31;
    for (int i = MW - 1; i >= 0; --i) {
        int src = i - L;
        if (src < 0) continue;
        uint64_t v = (uint64_t)a->w[src] << b;
        if (b && src - 1 >= 0) v |= (uint64_t)a->w[src - 1] >> (32 - b);
        t.w[i] = (uint32_t)v;
    }
    *r = t;
}
static int mw_cmp(const mw* a, const mw* b) {
    for (int i = MW - 1; i >= 0; --i)
        if (a->w[i] != b->w[i]) return a->w[i] < b->w[i] ? -1 : 1;
    return 0;
}
static void mw_sub(mw* a, const mw* b) { /* a -= b, a >= b */
    int64_t br = 0;
    for (int i = 0; i < MW; ++i) {
        int64_t x = (int64_t)a->w[i] - b->w[i] - br;
        br = x < 0;
        a->w[i] = (uint32_t)(x + (br ? ((int64_t)1 << 32) : 0));
    }
}
static u64 mw_extract(const mw* a, int lo, int nbits) { /* bits [lo, lo+nbits) of a, lo may be < 0 */
    u64 r = 0;
    for (int i = nbits - 1; i >= 0; --i) r = (r << 1) | (u64)mw_bit(a, lo + i);
    return r;
}

typedef struct { int p, qmin, emax; } fmt_t;
static const fmt_t F32 = {24, -149, 127};
static const fmt_t B16 = {8, -133, 127};

/* Rounded value sign * m * 2^e; m == 0 is zero. */
typedef struct { int sign; u64 m; int e; int overflow; } rounded;

static int rounded_eq(rounded a, rounded b) {
    if (a.overflow || b.overflow) return 0;
    if (a.m == 0 && b.m == 0) return 1;
    return a.sign == b.sign && a.m == b.m && a.e == b.e;
}

/* RN-even of the exact value mag * 2^ebase into f (mag != 0). */
static rounded round_mw(const mw* mag, int ebase, int sign, fmt_t f) {
    rounded r = {sign, 0, 0, 0};
    int bl = mw_bitlen(mag);
    if (!bl) return r;
    long k = (long)bl - 1 + ebase; /* floor(log2 value) */
    long qe = k - (f.p - 1);
    if (qe < f.qmin) qe = f.qmin;
    long lo = qe - ebase; /* bit index of the quantum */
    u64 q;
    int rb, st;
    if (lo >= 0) {
        q = mw_extract(mag, (int)lo, f.p + 1);
        rb = mw_bit(mag, (int)lo - 1);
        st = mw_any_below(mag, (int)lo - 1);
    } else {
        q = mw_extract(mag, 0, f.p + 1) << (-lo);
        rb = 0;
        st = 0;
    }
    if (rb && (st || (q & 1))) ++q;
    if (q == ((u64)1 << f.p)) {
        q >>= 1;
        ++qe;
    }
    if (q && qe + (63 - __builtin_clzll(q)) > f.emax) r.overflow = 1;
    r.m = q;
    r.e = (int)qe;
    return r;
}

/* RN-even of (a / b) * 2^E, a, b < 2^128, b > 0 (csrc/exact_attention_cpu.cpp:111-153). */
static rounded round_ratio(u128 a_, u128 b_, int E, int sign, fmt_t f) {
    rounded r = {sign, 0, 0, 0};
    if (a_ == 0) return r;
    mw a, b, t;
    mw_from_u128(&a, a_);
    mw_from_u128(&b, b_);
    int k = mw_bitlen(&a) - mw_bitlen(&b);
    if (k >= 0) {
        mw_shl(&t, &b, k);
        if (mw_cmp(&a, &t) < 0) --k;
    } else {
        mw_shl(&t, &a, -k);
        if (mw_cmp(&t, &b) < 0) --k;
    }
    long K = (long)k + E;
    if (K < (long)f.qmin - 1) return r;
    long qe = K - (f.p - 1);
    if (qe < f.qmin) qe = f.qmin;
    long s = (long)E - qe;
    mw n = a, d = b;
    if (s >= 0) mw_shl(&n, &a, (int)s);
    else mw_shl(&d, &b, (int)-s);
    u64 q = 0;
    for (int i = f.p + 1; i >= 0; --i) {
        mw_shl(&t, &d, i);
        if (mw_cmp(&n, &t) >= 0) {
            mw_sub(&n, &t);
            q |= (u64)1 << i;
        }
    }
    mw_shl(&t, &n, 1);
    int c = mw_cmp(&t, &d);
    if (c > 0 || (c == 0 && (q & 1))) ++q;
    if (q == ((u64)1 << f.p)) {
        q >>= 1;
        ++qe;
    }
    if (qe + (63 - __builtin_clzll(q)) > f.emax) r.overflow = 1;
    r.m = q;
    r.e = (int)qe;
    return r;
}

static uint32_t rounded_bits(rounded r, int fp32) {
    if (r.m == 0) return 0;
    int p = fp32 ? 24 : 8, qmin = fp32 ? -149 : -133;
    u64 m = r.m;
    int e = r.e;
    while (m < ((u64)1 << (p - 1)) && e > qmin) {
        m <<= 1;
        --e;
    }
    uint32_t field, frac;
    if (m < ((u64)1 << (p - 1))) {
        field = 0;
        frac = (uint32_t)m;
    } else {
        field = (uint32_t)(e - qmin + 1);
        frac = (uint32_t)(m - ((u64)1 << (p - 1)));
    }
    uint32_t sgn = r.sign < 0 ? 1u : 0u;
    return (sgn << (p - 1 + 8)) | (field << (p - 1)) | frac;
}

/* ------------------------------------------------------------------------------------------
 * Decoding (csrc/exact_attention_cpu.cpp:164-199)
 * ---------------------------------------------------------------------------------------- */
typedef struct { int32_t m, e; } dy;

static inline int decode_bf16(uint16_t b, dy* o) {
    int ex = (b >> 7) & 0xFF, fr = b & 0x7F, sg = (b & 0x8000) ? -1 : 1;
    if (ex == 0xFF) return 0;
    if (ex == 0) {
        o->m = sg * fr;
        o->e = -133;
    } else {
        o->m = sg * (fr | 0x80);
        o->e = ex - 134;
    }
    return 1;
}

static inline int decode_fp32_bits(uint32_t b, int32_t* m, int32_t* e) {
    int ex = (b >> 23) & 0xFF;
    int32_t fr = b & 0x7FFFFF;
    int sg = (b & 0x80000000u) ? -1 : 1;
    if (ex == 0xFF) return 0;
    if (ex == 0) {
        *m = sg * fr;
        *e = -149;
    } else {
        *m = sg * (fr | 0x800000);
        *e = ex - 150;
    }
    return 1;
}

static inline int ilog2_u64(u64 x) { return 63 - __builtin_clzll(x); }

/* ------------------------------------------------------------------------------------------
 * Exact score and logit. The reference windows the score into an int64 and certifies
 * (csrc/exact_attention_cpu.cpp:215-255); the oracle computes it exactly instead.
 * ---------------------------------------------------------------------------------------- */
#define SL 20              /* redundant int64 limbs, each weighting 2^(32*i + SEBASE) */
#define SEBASE (-266 - 32) /* below the smallest product exponent (-133) + (-133) */

/* Returns 0 if the logit overflows fp32 (a domain error), else 1 with t as fp32 bits. */
static int exact_logit(const dy* q, const dy* k, int d, int32_t am, int32_t ae, uint32_t* t_bits) {
    int64_t acc[SL];
    memset(acc, 0, sizeof(acc));
    int any = 0;
    for (int i = 0; i < d; ++i) {
        int64_t p = (int64_t)q[i].m * k[i].m;
        if (!p) continue;
        any = 1;
        int o = q[i].e + k[i].e - SEBASE;
        acc[o >> 5] += p << (o & 31); /* |p << 31| < 2^47; at most d adds per limb */
    }
    if (!any || am == 0) {
        *t_bits = 0;
        return 1;
    }
    /* normalise to two's complement 32-bit digits */
    uint32_t dig[SL + 2];
    int64_t c = 0;
    for (int i = 0; i < SL; ++i) {
        int64_t x = acc[i] + c;
        dig[i] = (uint32_t)x;
        c = x >> 32; /* arithmetic */
    }
    int neg = c < 0;
    /* magnitude */
    mw mag;
    mw_zero(&mag);
    if (!neg) {
        for (int i = 0; i < SL; ++i) mag.w[i] = dig[i];
    } else {
        uint64_t br = 1; /* -x = ~x + 1 */
        for (int i = 0; i < SL; ++i) {
            uint64_t v = (uint64_t)(uint32_t)~dig[i] + br;
            mag.w[i] = (uint32_t)v;
            br = v >> 32;
        }
    }
    /* times |alpha_m| */
    uint64_t am_abs = (uint64_t)(am < 0 ? -(int64_t)am : am);
    uint64_t carry = 0;
    for (int i = 0; i < MW; ++i) {
        uint64_t v = (uint64_t)mag.w[i] * am_abs + carry;
        mag.w[i] = (uint32_t)v;
        carry = v >> 32;
    }
    int sign = (neg ? -1 : 1) * (am < 0 ? -1 : 1);
    rounded r = round_mw(&mag, SEBASE + ae, sign, F32);
    if (r.overflow) return 0;
    *t_bits = rounded_bits(r, 1);
    return 1;
}

/* ------------------------------------------------------------------------------------------
 * Weights w = RN24(2^t) (docs/SPEC.md step 3). Own method: an integer interval enclosure of
 * 2^f at scale 2^126: 2^f = T[j] * exp(r ln 2), j = top 8 bits of f, with the 256 table
 * enclosures built once by the same series. Both ends of the enclosure round the same, or the
 * weight is reported undecided (the row is then flagged for the Python oracle).
 * ---------------------------------------------------------------------------------------- */
#define XS 126
/* floor / ceil of (a * b) >> 126 for a, b < 2^127 */
static u128 mulshr(u128 a, u128 b, int up) {
    u64 a1 = (u64)(a >> 64), a0 = (u64)a, b1 = (u64)(b >> 64), b0 = (u64)b;
    u128 p00 = (u128)a0 * b0, p01 = (u128)a0 * b1, p10 = (u128)a1 * b0, p11 = (u128)a1 * b1;
    /* 256-bit sum: (p11 << 128) + ((p01 + p10) << 64) + p00 */
    u128 mid = p01 + p10;
    u128 mid_c = mid < p01 ? 1 : 0; /* carry out of the 128-bit mid */
    u128 lo = p00 + (mid << 64);
    u128 lo_c = lo < p00 ? 1 : 0;
    u128 hi = p11 + (mid >> 64) + (mid_c << 64) + lo_c;
    /* result = (hi:lo) >> 126 */
    u128 res = (hi << 2) | (lo >> 126);
    if (up && (lo & (((u128)1 << 126) - 1))) ++res;
    return res;
}
static u128 divsmall(u128 a, u64 n, int up) {
    u128 q = a / n;
    if (up && q * n != a) ++q;
    return q;
}

/* ln2 * 2^126 enclosure; pinned against oracle/exact.py:ln2_enclosure by a test. */
static u128 LN2_LO, LN2_HI;
static u128 TLO[256], THI[256]; /* 2^(j/256) * 2^126 enclosures */
static int tables_ready = 0;
static pthread_mutex_t tables_mu = PTHREAD_MUTEX_INITIALIZER;

/* exp(x) * 2^126 enclosure for x in [xl, xh] * 2^-126, 0 <= x < 1. */
static void exp_encl(u128 xl, u128 xh, u128* lo, u128* hi) {
    u128 one = (u128)1 << XS;
    u128 s = 0, t = one;
    for (u64 n = 1; t; ++n) {
        s += t;
        t = divsmall(mulshr(t, xl, 0), n, 0);
    }
    *lo = s;
    s = 0;
    t = one;
    for (u64 n = 1;; ++n) {
        s += t;
        t = divsmall(mulshr(t, xh, 1), n, 1);
        if (t <= 1 && n > 3) {
            s += 2 * t + 2;
            break;
        }
    }
    *hi = s;
}

static void init_tables(void) {
    pthread_mutex_lock(&tables_mu);
    if (!tables_ready) {
        /* ln 2 = sum_k 2 / ((2k+1) 3^(2k+1)) at scale 2^126, floors and ceils, plus tail */
        /* floor(floor(a/b)/c) = floor(a/(bc)) and ceil(ceil(a/b)/c) = ceil(a/(bc)), so the
         * product (2k+1) 3^(2k+1), which would overflow, is never formed. */
        u128 one = (u128)1 << XS, lo = 0, hi = 0, p3 = 3;
        for (u64 k = 0;; ++k) {
            u128 a = 2 * one;
            u128 tl = (a / p3) / (2 * k + 1);
            u128 c1 = (a + p3 - 1) / p3;
            lo += tl;
            hi += (c1 + 2 * k) / (2 * k + 1);
            if (tl == 0) break; /* here 3^(2k+1) (2k+1) > 2^127 and p3 < 2^123 */
            p3 *= 9;
        }
        hi += 2; /* the tail after the first zero term is below 2^127 / (9 * 3^(2k+1) (2k+1)) < 1 */
        LN2_LO = lo;
        LN2_HI = hi;
        for (int j = 0; j < 256; ++j) {
            /* x = (j / 256) ln 2 */
            /* split to avoid overflowing 128 bits: floor/ceil of LN2 * j / 256 */
            u128 xl = (LN2_LO >> 8) * (u128)j + (((LN2_LO & 255) * (u128)j) >> 8);
            u128 xh = (LN2_HI >> 8) * (u128)j + (((LN2_HI & 255) * (u128)j + 255) >> 8);
            exp_encl(xl, xh, &TLO[j], &THI[j]);
        }
        tables_ready = 1;
    }
    pthread_mutex_unlock(&tables_mu);
}

/* Returns 1 and (M, E) if decided, 0 if undecided or |t| >= 2^30 (the reference flags those too,
 * csrc/exact_attention_cpu.cpp:262). */
static int weight(uint32_t t_bits, int32_t* M, i64* E) {
    int32_t tm = 0, te = 0;
    decode_fp32_bits(t_bits, &tm, &te);
    int field = (t_bits >> 23) & 0xFF;
    if (tm == 0 || field < 102) { /* |t| < 2^-25: RN24(2^t) = 1 */
        *M = 1 << 23;
        *E = -23;
        return 1;
    }
    if (field >= 127 + 30) return 0; /* |t| >= 2^30 */
    /* t = tm * 2^te with te >= -48 here; n = floor(t), f = F * 2^-48 */
    i64 n;
    u64 F;
    if (te >= 0) {
        n = (i64)tm << te;
        F = 0;
    } else {
        int s = -te;
        n = (i64)tm >> s; /* floor */
        i64 a = (i64)tm - (n << s);
        F = (u64)a << (48 - s);
    }
    if (F == 0) {
        *M = 1 << 23;
        *E = n - 23;
        return 1;
    }
    int j = (int)(F >> 40);
    u64 R = F & ((1ull << 40) - 1); /* r = R * 2^-48 < 2^-8 */
    /* x = r ln2 at scale 2^126: (R * LN2) >> 48 */
    u128 xl = mulshr((u128)R << 78, LN2_LO, 0); /* (R<<78)*LN2 >> 126 = R*LN2 >> 48 */
    u128 xh = mulshr((u128)R << 78, LN2_HI, 1);
    u128 el, eh;
    exp_encl(xl, xh, &el, &eh);
    u128 yl = mulshr(TLO[j], el, 0), yh = mulshr(THI[j], eh, 1);
    /* M = round(y * 2^23 / 2^126) */
    int sh = XS - 23;
    u128 half = (u128)1 << (sh - 1);
    u128 ql = (yl + half) >> sh, qh = (yh + half) >> sh;
    if (ql != qh) return 0;
    i64 e = n - 23;
    if (ql == ((u128)1 << 24)) {
        ql >>= 1;
        ++e;
    }
    *M = (int32_t)ql;
    *E = e;
    return 1;
}

/* ------------------------------------------------------------------------------------------
 * Partials (csrc/exact_attention_cpu.cpp:296-441 and src/exactattn/certified.py:145-246).
 * Accumulators are stored in 128 bits and checked against the configured width B (64 or 128).
 * ---------------------------------------------------------------------------------------- */
#define NEG_INF INT64_MIN

static inline i128 floor_shift(i128 m, i64 sh, int B, int* lost) {
    if (sh >= 0) {
        *lost = 0;
        return m << sh; /* headroom guaranteed by construction */
    }
    i64 s = -sh;
    if (s >= B - 1) {
        *lost = m != 0;
        return m < 0 ? -1 : 0;
    }
    i128 v = m >> s;
    *lost = (v << s) != m;
    return v;
}

static inline void rescale(i128* acc, u64* err, i64 s, int B) {
    if (s <= 0) return;
    int lost;
    *acc = floor_shift(*acc, -s, B, &lost);
    u64 e = s >= 64 ? (*err ? 1 : 0) : (*err >> s) + ((*err & ((1ull << s) - 1)) != 0);
    *err = e + (lost ? 1 : 0);
}

static inline int fits(i128 v, u64 err, int B) {
    u128 a = v < 0 ? (u128)(-(v + 1)) + 1 : (u128)v;
    u128 lim = (u128)1 << (B - 1);
    return a < lim && (u128)err < lim - a;
}

typedef struct {
    int empty;
    i64 R;
    i128 Z;
    u64 Zerr, count;
    i64* NR;
    i128* N;
    u64* Nerr;
} partial;

typedef struct { int d, dv, fz, fn, key_log2, B; } ctx;

static void partial_init(partial* p, int dv, i64* NR, i128* N, u64* Nerr) {
    p->empty = 1;
    p->R = 0;
    p->Z = 0;
    p->Zerr = 0;
    p->count = 0;
    p->NR = NR;
    p->N = N;
    p->Nerr = Nerr;
    for (int c = 0; c < dv; ++c) {
        NR[c] = NEG_INF;
        N[c] = 0;
        Nerr[c] = 0;
    }
}

static void partial_copy(partial* dst, const partial* src, int dv) {
    dst->empty = src->empty;
    dst->R = src->R;
    dst->Z = src->Z;
    dst->Zerr = src->Zerr;
    dst->count = src->count;
    memcpy(dst->NR, src->NR, sizeof(i64) * dv);
    memcpy(dst->N, src->N, sizeof(i128) * dv);
    memcpy(dst->Nerr, src->Nerr, sizeof(u64) * dv);
}

static int tile_partial(const ctx* c, const int32_t* M, const i64* Ew, const dy* const* vrows, int n,
                        partial* p) {
    if (n == 0) return 1;
    p->empty = 0;
    p->count = (u64)n;
    i64 R = NEG_INF;
    for (int j = 0; j < n; ++j)
        if (Ew[j] + 23 > R) R = Ew[j] + 23;
    p->R = R;
    for (int j = 0; j < n; ++j) {
        int lost;
        p->Z += floor_shift((i128)M[j], Ew[j] - (R - c->fz), c->B, &lost);
        p->Zerr += (u64)lost;
    }
    if (!fits(p->Z, p->Zerr, c->B)) return 0;
    for (int ch = 0; ch < c->dv; ++ch) {
        i64 NR = NEG_INF;
        for (int j = 0; j < n; ++j) {
            int32_t m = vrows[j][ch].m;
            if (!m) continue;
            i64 L = Ew[j] + 23 + 1 + vrows[j][ch].e + ilog2_u64((u64)(m < 0 ? -m : m));
            if (L > NR) NR = L;
        }
        if (NR == NEG_INF) continue;
        p->NR[ch] = NR;
        i64 base = NR - c->fn;
        i128 acc = 0;
        u64 err = 0;
        for (int j = 0; j < n; ++j) {
            int32_t m = vrows[j][ch].m;
            if (!m) continue;
            int lost;
            acc += floor_shift((i128)((i64)M[j] * m), Ew[j] + vrows[j][ch].e - base, c->B, &lost);
            err += (u64)lost;
        }
        if (!fits(acc, err, c->B)) return 0;
        p->N[ch] = acc;
        p->Nerr[ch] = err;
    }
    return 1;
}

static int merge_into(const ctx* c, partial* a, const partial* b) {
    if (b->empty) return 1;
    if (a->empty) {
        partial_copy(a, b, c->dv);
        return 1;
    }
    a->count += b->count;
    if (a->count > ((u64)1 << c->key_log2)) return 0;
    i64 R = a->R > b->R ? a->R : b->R;
    i128 za = a->Z, zb = b->Z;
    u64 ea = a->Zerr, eb = b->Zerr;
    rescale(&za, &ea, R - a->R, c->B);
    rescale(&zb, &eb, R - b->R, c->B);
    a->R = R;
    a->Z = za + zb;
    a->Zerr = ea + eb;
    if (!fits(a->Z, a->Zerr, c->B)) return 0;
    for (int ch = 0; ch < c->dv; ++ch) {
        i64 ra = a->NR[ch], rb = b->NR[ch];
        if (rb == NEG_INF) continue;
        if (ra == NEG_INF) {
            a->NR[ch] = rb;
            a->N[ch] = b->N[ch];
            a->Nerr[ch] = b->Nerr[ch];
            continue;
        }
        i64 ref = ra > rb ? ra : rb;
        i128 xa = a->N[ch], xb = b->N[ch];
        u64 eA = a->Nerr[ch], eB = b->Nerr[ch];
        rescale(&xa, &eA, ref - ra, c->B);
        rescale(&xb, &eB, ref - rb, c->B);
        a->NR[ch] = ref;
        a->N[ch] = xa + xb;
        a->Nerr[ch] = eA + eB;
        if (!fits(a->N[ch], a->Nerr[ch], c->B)) return 0;
    }
    return 1;
}

static u128 mag128(i128 v) { return v < 0 ? (u128)(-v) : (u128)v; }

/* csrc/exact_attention_cpu.cpp:450-490 */
static int finalize(const ctx* c, const partial* p, int fp32_out, void* out_row) {
    uint16_t* o16 = (uint16_t*)out_row;
    uint32_t* o32 = (uint32_t*)out_row;
    for (int ch = 0; ch < c->dv; ++ch) {
        if (fp32_out) o32[ch] = 0;
        else o16[ch] = 0;
    }
    if (p->empty) return 1;
    fmt_t f = fp32_out ? F32 : B16;
    i64 zunit = p->R - c->fz;
    i128 Zlo = p->Z, Zhi = p->Z + (i128)p->Zerr;
    if (Zlo <= 0) return 0;
    for (int ch = 0; ch < c->dv; ++ch) {
        if (p->NR[ch] == NEG_INF) continue;
        i64 nunit = p->NR[ch] - c->fn;
        i128 Nlo = p->N[ch], Nhi = p->N[ch] + (i128)p->Nerr[ch];
        i128 ln, ld, hn, hd;
        if (Nlo >= 0) {
            ln = Nlo; ld = Zhi; hn = Nhi; hd = Zlo;
        } else if (Nhi <= 0) {
            ln = Nlo; ld = Zlo; hn = Nhi; hd = Zhi;
        } else {
            ln = Nlo; ld = Zlo; hn = Nhi; hd = Zlo;
        }
        i64 sh = nunit - zunit;
        if (sh > 100000 || sh < -100000) return 0;
        rounded rl = round_ratio(mag128(ln), (u128)ld, (int)sh, ln < 0 ? -1 : 1, f);
        rounded rh = round_ratio(mag128(hn), (u128)hd, (int)sh, hn < 0 ? -1 : 1, f);
        if (!rounded_eq(rl, rh)) return 0;
        uint32_t bits = rounded_bits(rl, fp32_out);
        if (fp32_out) o32[ch] = bits;
        else o16[ch] = (uint16_t)bits;
    }
    return 1;
}

/* ------------------------------------------------------------------------------------------
 * Row engine. A row is given by its decoded q and the list of its visible key rows.
 * ---------------------------------------------------------------------------------------- */
typedef struct {
    int d, dv, fp32_out, tile, splits;
    uint32_t alpha_bits;
    int32_t am, ae;
    u64 order_seed;
    ctx c;
} engine;

typedef struct {
    dy* qd;
    dy* kd;  /* one decoded key row */
    int32_t* M;
    i64* E;
    const dy** vrows;
    dy* vdec; /* decoded value rows, n * dv */
    partial* parts;
    i64 *pNR;
    i128* pN;
    u64* pNerr;
    partial tp, total;
    i64 *tNR, *totNR;
    i128 *tN, *totN;
    u64 *tNerr, *totNerr;
    int* order;
    i64 cap_keys, cap_splits;
} scratch;

static void scratch_free(scratch* s) {
    free(s->qd); free(s->kd); free(s->M); free(s->E); free(s->vrows); free(s->vdec);
    free(s->parts); free(s->pNR); free(s->pN); free(s->pNerr);
    free(s->tNR); free(s->totNR); free(s->tN); free(s->totN); free(s->tNerr); free(s->totNerr);
    free(s->order);
    memset(s, 0, sizeof(*s));
}

static int scratch_reserve(scratch* s, const engine* g, i64 n) {
    int d = g->d, dv = g->dv;
    if (!s->qd) {
        s->qd = malloc(sizeof(dy) * d);
        s->kd = malloc(sizeof(dy) * d);
        s->tNR = malloc(sizeof(i64) * dv); s->tN = malloc(sizeof(i128) * dv); s->tNerr = malloc(sizeof(u64) * dv);
        s->totNR = malloc(sizeof(i64) * dv); s->totN = malloc(sizeof(i128) * dv); s->totNerr = malloc(sizeof(u64) * dv);
        i64 S = g->splits;
        s->parts = malloc(sizeof(partial) * S);
        s->pNR = malloc(sizeof(i64) * dv * S); s->pN = malloc(sizeof(i128) * dv * S); s->pNerr = malloc(sizeof(u64) * dv * S);
        s->order = malloc(sizeof(int) * S);
        s->cap_splits = S;
        if (!s->qd || !s->kd || !s->parts || !s->pN || !s->order) return 0;
    }
    if (n > s->cap_keys) {
        i64 c = n + 1024;
        free(s->M); free(s->E); free(s->vrows); free(s->vdec);
        s->M = malloc(sizeof(int32_t) * c);
        s->E = malloc(sizeof(i64) * c);
        s->vrows = malloc(sizeof(dy*) * c);
        s->vdec = malloc(sizeof(dy) * c * dv);
        s->cap_keys = c;
        if (!s->M || !s->E || !s->vrows || !s->vdec) return 0;
    }
    return 1;
}

static u64 splitmix(u64* x) {
    u64 z = (*x += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* stats[0..2] += score, weight, final fallbacks (csrc/exact_attention_cpu.cpp:580-584) */
static uint8_t run_row(const engine* g, scratch* s, i64 row, const uint16_t* q, const uint16_t* const* krows,
                       const uint16_t* const* vsrc, i64 n, void* orow, i64* stats) {
    int d = g->d, dv = g->dv;
    const ctx* c = &g->c;
    uint8_t flag = 0;
    for (int i = 0; i < dv; ++i) {
        if (g->fp32_out) ((uint32_t*)orow)[i] = 0;
        else ((uint16_t*)orow)[i] = 0;
    }
    for (int i = 0; i < d; ++i)
        if (!decode_bf16(q[i], &s->qd[i])) flag = 2;
    /* non-finite keys/values anywhere in the visible set make the row a domain error */
    for (i64 j = 0; j < n && flag != 2; ++j) {
        for (int i = 0; i < d; ++i)
            if (((krows[j][i] >> 7) & 0xFF) == 0xFF) flag = 2;
        for (int i = 0; i < dv; ++i)
            if (((vsrc[j][i] >> 7) & 0xFF) == 0xFF) flag = 2;
    }
    if (flag) return flag;
    for (i64 j = 0; j < n; ++j) {
        for (int i = 0; i < d; ++i) decode_bf16(krows[j][i], &s->kd[i]);
        uint32_t tb;
        if (!exact_logit(s->qd, s->kd, d, g->am, g->ae, &tb)) return 2; /* fp32 logit overflow */
        if (!weight(tb, &s->M[j], &s->E[j])) {
            stats[1]++;
            return 1;
        }
        dy* vd = s->vdec + j * dv;
        for (int i = 0; i < dv; ++i) decode_bf16(vsrc[j][i], &vd[i]);
        s->vrows[j] = vd;
    }
    int S = (int)(g->splits < (n > 1 ? n : 1) ? g->splits : (n > 1 ? n : 1));
    if (S < 1) S = 1;
    for (int k = 0; k < S; ++k)
        partial_init(&s->parts[k], dv, s->pNR + (i64)k * dv, s->pN + (i64)k * dv, s->pNerr + (i64)k * dv);
    partial_init(&s->tp, dv, s->tNR, s->tN, s->tNerr);
    for (int k = 0; k < S && !flag; ++k) {
        i64 cb = n * k / S, ce = n * (k + 1) / S;
        for (i64 t0 = cb; t0 < ce && !flag; t0 += g->tile) {
            i64 t1 = t0 + g->tile < ce ? t0 + g->tile : ce;
            partial_init(&s->tp, dv, s->tNR, s->tN, s->tNerr);
            if (!tile_partial(c, &s->M[t0], &s->E[t0], &s->vrows[t0], (int)(t1 - t0), &s->tp) ||
                !merge_into(c, &s->parts[k], &s->tp))
                flag = 1;
        }
    }
    for (int k = 0; k < S; ++k) s->order[k] = k;
    u64 st = g->order_seed ^ ((u64)row * 0x9E3779B97F4A7C15ull);
    for (int k = S - 1; k > 0; --k) {
        int j = (int)(splitmix(&st) % (u64)(k + 1));
        int tmp = s->order[k];
        s->order[k] = s->order[j];
        s->order[j] = tmp;
    }
    partial_init(&s->total, dv, s->totNR, s->totN, s->totNerr);
    for (int k = 0; k < S && !flag; ++k)
        if (!merge_into(c, &s->total, &s->parts[s->order[k]])) flag = 1;
    if (!flag && !finalize(c, &s->total, g->fp32_out, orow)) {
        flag = 1;
        stats[2]++;
    }
    if (flag == 1)
        for (int i = 0; i < dv; ++i) {
            if (g->fp32_out) ((uint32_t*)orow)[i] = 0;
            else ((uint16_t*)orow)[i] = 0;
        }
    return flag;
}

static int engine_init(engine* g, int d, int dv, uint32_t alpha_bits, int fp32_out, int acc_bits, int tile,
                       int splits, u64 order_seed, i64 maxn) {
    if (d <= 0 || d > 1024 || dv <= 0 || tile <= 0 || splits <= 0) return -1;
    if (acc_bits != 64 && acc_bits != 128) return -2;
    g->d = d;
    g->dv = dv;
    g->fp32_out = fp32_out;
    g->tile = tile;
    g->splits = splits;
    g->alpha_bits = alpha_bits;
    g->order_seed = order_seed;
    if (!decode_fp32_bits(alpha_bits, &g->am, &g->ae)) return -3;
    int key_log2 = 0;
    if (maxn < 1) maxn = 1;
    while (((i64)1 << key_log2) < maxn) ++key_log2;
    g->c.d = d;
    g->c.dv = dv;
    g->c.key_log2 = key_log2;
    g->c.B = acc_bits;
    g->c.fz = g->c.fn = acc_bits - 2 - key_log2;
    init_tables();
    return 0;
}

/* ------------------------------------------------------------------------------------------
 * CSR entry point: the reference C ABI (csrc/exact_attention_cpu.cpp:585-628).
 * ---------------------------------------------------------------------------------------- */
typedef struct {
    const engine* g;
    const uint16_t *q, *k, *v;
    const i64 *row_ptr, *key_idx;
    void* out;
    uint8_t* flags;
    i64 r0, r1;
    i64 stats[3];
    int ok;
} csr_job;

static void* csr_worker(void* arg) {
    csr_job* J = (csr_job*)arg;
    const engine* g = J->g;
    scratch s;
    memset(&s, 0, sizeof(s));
    const uint16_t** kr = NULL;
    const uint16_t** vr = NULL;
    i64 cap = 0;
    J->ok = 1;
    size_t osz = g->fp32_out ? 4 : 2;
    for (i64 r = J->r0; r < J->r1; ++r) {
        i64 b = J->row_ptr[r], n = J->row_ptr[r + 1] - b;
        if (!scratch_reserve(&s, g, n)) { J->ok = 0; break; }
        if (n > cap) {
            cap = n + 1024;
            free(kr); free(vr);
            kr = malloc(sizeof(*kr) * cap);
            vr = malloc(sizeof(*vr) * cap);
        }
        for (i64 j = 0; j < n; ++j) {
            i64 key = J->key_idx[b + j];
            kr[j] = J->k + key * g->d;
            vr[j] = J->v + key * g->dv;
        }
        J->flags[r] = run_row(g, &s, r, J->q + r * g->d, kr, vr, n, (char*)J->out + (size_t)r * g->dv * osz,
                              J->stats);
    }
    free(kr); free(vr);
    scratch_free(&s);
    return NULL;
}

int ea_attention_cpu(const uint16_t* q, int64_t rows, int d, const uint16_t* k, const uint16_t* v, int64_t nkeys,
                     int dv, float alpha, const int64_t* row_ptr, const int64_t* key_idx, int fp32_out,
                     int acc_bits, int tile, int splits, uint64_t order_seed, int nthreads, void* out,
                     uint8_t* flags, int64_t* stats) {
    (void)nkeys;
    uint32_t ab;
    memcpy(&ab, &alpha, 4);
    i64 maxn = 1;
    for (i64 r = 0; r < rows; ++r)
        if (row_ptr[r + 1] - row_ptr[r] > maxn) maxn = row_ptr[r + 1] - row_ptr[r];
    engine g;
    int rc = engine_init(&g, d, dv, ab, fp32_out, acc_bits, tile, splits, order_seed, maxn);
    if (rc) return rc;
    int T = nthreads > 0 ? nthreads : 1;
    if (T > rows) T = rows > 0 ? (int)rows : 1;
    csr_job* jobs = calloc(T, sizeof(csr_job));
    pthread_t* th = calloc(T, sizeof(pthread_t));
    for (int i = 0; i < T; ++i) {
        jobs[i] = (csr_job){&g, q, k, v, row_ptr, key_idx, out, flags, rows * i / T, rows * (i + 1) / T, {0, 0, 0}, 1};
        pthread_create(&th[i], NULL, csr_worker, &jobs[i]);
    }
    int ok = 1;
    for (int i = 0; i < T; ++i) {
        pthread_join(th[i], NULL);
        for (int j = 0; j < 3; ++j) stats[j] += jobs[i].stats[j];
        ok &= jobs[i].ok;
    }
    free(jobs);
    free(th);
    return ok ? 0 : -4;
}

/* Exposed for unit tests: csrc/exact_attention_cpu.cpp:632-638. Returns bits (fp32 or bf16). */
uint32_t oracle_round_ratio_bits(uint64_t a_hi, uint64_t a_lo, uint64_t b_hi, uint64_t b_lo, int E, int neg, int fp32,
                                 int* overflow) {
    u128 a = ((u128)a_hi << 64) | a_lo, b = ((u128)b_hi << 64) | b_lo;
    rounded r = round_ratio(a, b, E, neg ? -1 : 1, fp32 ? F32 : B16);
    *overflow = r.overflow;
    return r.overflow ? 0 : rounded_bits(r, fp32);
}

/* Exposed for unit tests: weights for fp32 t bits. Returns 1 if decided. */
int oracle_weight(uint32_t t_bits, int32_t* M, int64_t* E) {
    init_tables();
    return weight(t_bits, M, E);
}

/* Exposed for unit tests: t = RN32(alpha * q.k) bits; returns 0 on overflow. */
int oracle_logit(const uint16_t* q, const uint16_t* k, int d, uint32_t alpha_bits, uint32_t* t_bits) {
    dy qd[1024], kd[1024];
    for (int i = 0; i < d; ++i) {
        decode_bf16(q[i], &qd[i]);
        decode_bf16(k[i], &kd[i]);
    }
    int32_t am = 0, ae = 0;
    decode_fp32_bits(alpha_bits, &am, &ae);
    return exact_logit(qd, kd, d, am, ae, t_bits);
}

void oracle_ln2(uint64_t* lo_hi_lo_hi) {
    init_tables();
    lo_hi_lo_hi[0] = (u64)(LN2_LO >> 64);
    lo_hi_lo_hi[1] = (u64)LN2_LO;
    lo_hi_lo_hi[2] = (u64)(LN2_HI >> 64);
    lo_hi_lo_hi[3] = (u64)LN2_HI;
}

/* ------------------------------------------------------------------------------------------
 * Serving-geometry entry point. Same field meaning as the GPU library's ea_geometry.
 * ---------------------------------------------------------------------------------------- */
typedef struct {
    int32_t num_seqs, num_tokens, num_q_heads, num_kv_heads, head_dim, head_dim_v;
    int64_t q_seq_stride, q_tok_stride, q_head_stride;
    int64_t o_seq_stride, o_tok_stride, o_head_stride;
    int64_t k_page_stride, k_slot_stride, k_head_stride;
    int64_t v_page_stride, v_slot_stride, v_head_stride;
    int32_t page_size, block_table_stride, max_seq_len, pad0;
} geom;

typedef struct {
    const uint16_t *q, *k, *v;
    const int32_t *seq_len, *kv_len, *block_table;
    const int64_t* block_table_offset;
    const uint64_t* tree_mask;
    const int32_t* tree_base;
    void* out;
    uint8_t* flags;
} gbufs;

typedef struct {
    const engine* g;
    const geom* G;
    const gbufs* Bf;
    i64 r0, r1;
    i64 stats[3];
    int ok;
} geom_job;

static inline i64 key_row(const geom* G, const gbufs* Bf, i64 b, i64 n, int kv_is_v, int h) {
    i64 page, slot;
    if (Bf->block_table) {
        i64 off = Bf->block_table_offset ? Bf->block_table_offset[b] : b * (i64)G->block_table_stride;
        page = Bf->block_table[off + n / G->page_size];
        slot = n % G->page_size;
    } else {
        page = b;
        slot = n;
    }
    if (kv_is_v) return page * G->v_page_stride + slot * G->v_slot_stride + (i64)h * G->v_head_stride;
    return page * G->k_page_stride + slot * G->k_slot_stride + (i64)h * G->k_head_stride;
}

static void* geom_worker(void* arg) {
    geom_job* J = (geom_job*)arg;
    const engine* g = J->g;
    const geom* G = J->G;
    const gbufs* Bf = J->Bf;
    scratch s;
    memset(&s, 0, sizeof(s));
    const uint16_t** kr = NULL;
    const uint16_t** vr = NULL;
    i64 cap = 0;
    J->ok = 1;
    size_t osz = g->fp32_out ? 4 : 2;
    int T = G->num_tokens, Hq = G->num_q_heads, grp = G->num_q_heads / G->num_kv_heads;
    for (i64 r = J->r0; r < J->r1; ++r) {
        i64 b = r / ((i64)T * Hq), t = (r / Hq) % T, hq = r % Hq;
        int hk = (int)(hq / grp);
        i64 tok = b * T + t;
        /* visible keys: the prefix below min(kv_len, seq_len) and the tree keys at or past it and
           below seq_len, each key once (the serving geometry's definition) */
        i64 slen = Bf->seq_len[b];
        i64 L = Bf->kv_len[tok];
        L = L < 0 ? 0 : (L < slen ? L : slen);
        uint64_t mask = 0;
        if (Bf->tree_mask) {
            i64 tb = Bf->tree_base[b], lo = L - tb, hi = slen - tb;
            lo = lo < 0 ? 0 : (lo > 64 ? 64 : lo);
            hi = hi < 0 ? 0 : (hi > 64 ? 64 : hi);
            if (hi > lo) {
                uint64_t below_hi = hi >= 64 ? ~0ull : ((1ull << hi) - 1);
                uint64_t below_lo = lo >= 64 ? ~0ull : ((1ull << lo) - 1);
                mask = Bf->tree_mask[tok] & below_hi & ~below_lo;
            }
        }
        i64 n = L + __builtin_popcountll(mask);
        if (!scratch_reserve(&s, g, n)) { J->ok = 0; break; }
        if (n > cap) {
            cap = n + 1024;
            free(kr); free(vr);
            kr = malloc(sizeof(*kr) * cap);
            vr = malloc(sizeof(*vr) * cap);
        }
        i64 j = 0;
        for (i64 key = 0; key < L; ++key, ++j) {
            kr[j] = Bf->k + key_row(G, Bf, b, key, 0, hk);
            vr[j] = Bf->v + key_row(G, Bf, b, key, 1, hk);
        }
        for (int i = 0; i < 64; ++i)
            if (mask >> i & 1) {
                i64 key = Bf->tree_base[b] + i;
                kr[j] = Bf->k + key_row(G, Bf, b, key, 0, hk);
                vr[j] = Bf->v + key_row(G, Bf, b, key, 1, hk);
                ++j;
            }
        const uint16_t* qrow = Bf->q + b * G->q_seq_stride + t * G->q_tok_stride + hq * G->q_head_stride;
        char* orow = (char*)Bf->out + (size_t)(b * G->o_seq_stride + t * G->o_tok_stride + hq * G->o_head_stride) * osz;
        Bf->flags[r] = run_row(g, &s, r, qrow, kr, vr, n, orow, J->stats);
    }
    free(kr); free(vr);
    scratch_free(&s);
    return NULL;
}

/* Rows are enumerated (seq, token, q head) in that order; flags has one entry per row. */
int oracle_attention_geom(const geom* G, const gbufs* Bf, uint32_t alpha_bits, int fp32_out, int acc_bits, int tile,
                          int splits, uint64_t order_seed, int nthreads, int64_t* stats) {
    if (G->num_kv_heads <= 0 || G->num_q_heads % G->num_kv_heads) return -1;
    if (Bf->tree_mask && !Bf->tree_base) return -1;
    i64 rows = (i64)G->num_seqs * G->num_tokens * G->num_q_heads;
    i64 maxn = 1;
    for (i64 tok = 0; tok < (i64)G->num_seqs * G->num_tokens; ++tok) {
        i64 n = Bf->kv_len[tok] + (Bf->tree_mask ? __builtin_popcountll(Bf->tree_mask[tok]) : 0);
        if (n > maxn) maxn = n;
    }
    engine g;
    int rc = engine_init(&g, G->head_dim, G->head_dim_v, alpha_bits, fp32_out, acc_bits, tile, splits, order_seed,
                         maxn);
    if (rc) return rc;
    int T = nthreads > 0 ? nthreads : 1;
    if (T > rows) T = rows > 0 ? (int)rows : 1;
    geom_job* jobs = calloc(T, sizeof(geom_job));
    pthread_t* th = calloc(T, sizeof(pthread_t));
    for (int i = 0; i < T; ++i) {
        jobs[i] = (geom_job){&g, G, Bf, rows * i / T, rows * (i + 1) / T, {0, 0, 0}, 1};
        pthread_create(&th[i], NULL, geom_worker, &jobs[i]);
    }
    int ok = 1;
    for (int i = 0; i < T; ++i) {
        pthread_join(th[i], NULL);
        for (int j = 0; j < 3; ++j) stats[j] += jobs[i].stats[j];
        ok &= jobs[i].ok;
    }
    free(jobs);
    free(th);
    return ok ? 0 : -4;
}
