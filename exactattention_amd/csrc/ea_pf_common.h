// Device helpers of the int8-MFMA prefill kernel (ea_prefill.hip, 32-row blocks): tile DMA and
// barrier primitives, the score MFMAs and their fp64 fold, the branch-free certified logit and
// weight, and the exact per-pair path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ea_params.h"

namespace ea {
namespace pf {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr double PF_U = 0x1p-53 * (1.0 + 0x1p-28);
// 1.5 * 2^52 + 0x8080808080: y = Wf + this has the biased digits of Wf in its low 40 bits
constexpr double PF_C40 = 6755399441055744.0 + (double)0x8080808080ull;

template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// global row index of local row lr of segment (b, hk)
__device__ __forceinline__ int64_t seg_row(const Params& P, int64_t b, int hk, int lr, int* t_out) {
    int t = lr / P.grp, gi = lr % P.grp;
    *t_out = t;
    return row_index(P, b, t, hk * P.grp + gi);
}

// ------------------------------------------------------------------------------------------------
// w = RN24(2^t) = M 2^E for an exact fp32 t (bits), from the fp64 tables (T1 pre-scaled by 2^23)
// and the cubic; false when undecided or |t| >= 2^30 (the 128-bit enclosure decides those).
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ bool table_weight(uint32_t tbits, const double* T1s, const double* T2, int* Mout,
                                             int* Eout) {
    const uint32_t field = (tbits >> 23) & 0xFF;
    if (field < 102) {  // |t| < 2^-25: 2^t rounds to 1
        *Mout = 1 << 23;
        *Eout = -23;
        return true;
    }
    if (field >= 127 + 30) return false;
    const double c1 = u64_as_f64(EA_C_BITS[0]), c2 = u64_as_f64(EA_C_BITS[1]), c3 = u64_as_f64(EA_C_BITS[2]);
    const double d0 = (double)__uint_as_float(tbits);
    const double fl = floor(d0);
    const double f = d0 - fl;
    const int i = ((int)(f * 65536.0)) & 0xFFFF;
    const double rr = __fma_rn(-(double)i, 0x1p-16, f);
    const double poly = rr * __fma_rn(rr, __fma_rn(rr, c3, c2), c1);
    const double aa = T1s[i >> 8] * T2[i & 255];
    const double Y = __fma_rn(aa, poly, aa);
    const double Yr = (Y + 0x1.8p52) - 0x1.8p52;
    *Mout = (int)Yr;
    *Eout = (int)fl - 23;
    return fabs(Y - Yr) <= 0.5 - 0x1p-26;
}

// ------------------------------------------------------------------------------------------------
// The exact decision for one pair the fast path left undecided (the prefill kernel's cold path):
// t = RN32(alpha s) from the exact score, then w = RN24(2^t) from the fp64 tables or, when they
// cannot decide, the 128-bit enclosure. mode 0: the score from the digit planes, q row qrow (LDS,
// chunk c at c ^ qsw) and K row krow (the tile in global memory, chunk c at c ^ ksw), with
// D_st = sum_i q_s,i k_t,i by v_dot4 (|D| <= 128 x 2^14), equal weights s + t summed in int32
// (<= 4 x 2^21), S = sum_k acc_k 256^k in 128 bits and t = RN32(am S 2^eS); mode 1: from the bf16
// rows qr, kr (elements rounded at slicing) by TwoSum with a certified logit, the rows read 32
// elements at a time in 16-byte loads when both are 16-byte aligned (one memory round trip per
// batch instead of one per element); mode 2: q holds NaN/inf (no score). Returns (status, M, E):
// 0 w = M 2^E, 2 domain error, 3 score not certified, 4 weight not certified.
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ int3 pf_cold_pair(int mode, const uint8_t* qrow, int qsw, const uint8_t* krow, int ksw,
                                          const uint16_t* qr, const uint16_t* kr, int32_t am, int eS, double alpha,
                                          const double* T1s, const double* T2) {
    uint32_t tbits = 0;
    int ls = 3;
    if (mode == 0) {
        int D[4][4];
#pragma unroll
        for (int sq = 0; sq < 4; ++sq)
#pragma unroll
            for (int tk = 0; tk < 4; ++tk) D[sq][tk] = 0;
        for (int c16 = 0; c16 < 8; ++c16) {
            uint4 qc[4], kc[4];
#pragma unroll
            for (int sp = 0; sp < 4; ++sp) {
                qc[sp] = *(const uint4*)(qrow + (((8 * sp + c16) ^ qsw) << 4));
                kc[sp] = *(const uint4*)(krow + 8192 * sp + ((c16 ^ ksw) << 4));
            }
#pragma unroll
            for (int sq = 0; sq < 4; ++sq)
#pragma unroll
                for (int tk = 0; tk < 4; ++tk) {
                    int d = D[sq][tk];
                    d = __builtin_amdgcn_sdot4((int)qc[sq].x, (int)kc[tk].x, d, false);
                    d = __builtin_amdgcn_sdot4((int)qc[sq].y, (int)kc[tk].y, d, false);
                    d = __builtin_amdgcn_sdot4((int)qc[sq].z, (int)kc[tk].z, d, false);
                    D[sq][tk] = __builtin_amdgcn_sdot4((int)qc[sq].w, (int)kc[tk].w, d, false);
                }
        }
        i128 S = 0;
#pragma unroll
        for (int k = 6; k >= 0; --k) {
            int acc = 0;
#pragma unroll
            for (int sq = 0; sq < 4; ++sq)
                if (k - sq >= 0 && k - sq < 4) acc += D[sq][k - sq];
            S = S * 256 + (i128)acc;
        }
        ls = rn32_prod(am, S, eS, &tbits);
    } else if (mode == 1) {
        double ss = 0.0, es = 0.0, ea = 0.0;
        auto acc2 = [&](uint32_t qw, uint32_t kw) __attribute__((always_inline)) {
            double e0;
            ss = two_sum(ss, (double)__uint_as_float(qw << 16) * (double)__uint_as_float(kw << 16), &e0);
            es += e0;
            ea += fabs(e0);
            ss = two_sum(ss, (double)__uint_as_float(qw & 0xFFFF0000u) * (double)__uint_as_float(kw & 0xFFFF0000u), &e0);
            es += e0;
            ea += fabs(e0);
        };
        if ((((uintptr_t)qr | (uintptr_t)kr) & 15) == 0) {
#pragma unroll 1
            for (int c0 = 0; c0 < 128; c0 += 32) {
                uint4 qv[4], kv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    qv[u] = *(const uint4*)(qr + c0 + 8 * u);
                    kv[u] = *(const uint4*)(kr + c0 + 8 * u);
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    acc2(qv[u].x, kv[u].x);
                    acc2(qv[u].y, kv[u].y);
                    acc2(qv[u].z, kv[u].z);
                    acc2(qv[u].w, kv[u].w);
                }
            }
        } else {
#pragma unroll 1
            for (int c = 0; c < 128; ++c) {
                double e0;
                ss = two_sum(ss, (double)__uint_as_float((uint32_t)qr[c] << 16) * (double)__uint_as_float((uint32_t)kr[c] << 16),
                             &e0);
                es += e0;
                ea += fabs(e0);
            }
        }
        ls = (ss == 0.0 && es == 0.0 && ea == 0.0) ? 1 : logit_cert(alpha, ss, es, ea * 0x1p-44, &tbits);
        if (ls == 1) tbits = 0;
    }
    int32_t M = 0, E = 0;
    if (ls == 2) return make_int3(2, M, E);
    if (ls == 3) return make_int3(3, M, E);
    if (table_weight(tbits, T1s, T2, &M, &E)) return make_int3(0, M, E);
    int32_t M2 = 0;
    int64_t E2 = 0;
    if (weight_wide(tbits, &M2, &E2) == 0 && E2 > -(1LL << 30) && E2 < (1LL << 30)) return make_int3(0, M2, (int32_t)E2);
    return make_int3(4, M, E);
}

// ------------------------------------------------------------------------------------------------
// Branch-free certified t = RN32(alpha s) and w = RN24(2^t) = M 2^E for 4 pairs in lock step
// (independent chains the scheduler interleaves). xs: fp64 scores in units 2^lsbq; a = alpha 2^lsbq;
// adel >= (1 + 2^-50) |a| |xs - exact| (the score bound with its rounding slack). p + pe = a xs
// exactly (FMA). The interval around p + pe rounds to t0 = RN32(p) when |p + pe - t0| + adel is
// below the smaller half gap next to t0 (2^(e - 24) for |t0| in [2^e, 2^(e+1)), 2^(e - 25) when
// |t0| is a power of two: the gap below it is half as wide); |alpha s| <= 2^-25 gives w = 1. 2^f from the
// fp64 tables (T1 pre-scaled by 2^23) and the cubic in r = f - j 2^-16, evaluated on
// rr = 2^16 r with the coefficients scaled by 2^-16, 2^-32, 2^-48 (every intermediate is the
// unscaled evaluation times a power of two: the same bits); rounded to an integer by adding and
// subtracting 1.5 * 2^52; certified when |Y - RN(Y)| <= 1/2 - 2^-26 (the fp64 evaluation error
// is below 2^-26.9). ok[i] false: the exact path decides.
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ void cert4(const double (&xs)[4], const double (&adel)[4], double a, const double* T1s,
                                      const double* T2, int (&M)[4], int (&E)[4], bool (&ok)[4]) {
    const double c1 = u64_as_f64(EA_C_BITS[0]) * 0x1p-16, c2 = u64_as_f64(EA_C_BITS[1]) * 0x1p-32,
                 c3 = u64_as_f64(EA_C_BITS[2]) * 0x1p-48;
    double d0[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const double p = a * xs[i];
        const double pe = __fma_rn(a, xs[i], -p);
        const float tf = (float)p;
        const double t0 = (double)tf;
        const double r = (p - t0) + pe;  // p - t0 is exact; one rounding, covered by 2^-50 below
        const double at = fabs(t0);
        // the smaller half gap next to t0: 2^(e - 24), or 2^(e - 25) when |t0| = 2^e
        const uint32_t hx = (uint32_t)__double2hiint(t0) & 0x7FF00000u;
        const uint32_t hsh = (__float_as_uint(tf) & 0x7FFFFFu) ? (24u << 20) : (25u << 20);
        const double h = __hiloint2double((int)(hx - hsh), 0);
        const bool tiny = fabs(p) + fabs(pe) + adel[i] <= 0x1p-25 * (1.0 - 0x1p-20);
        const bool inner = (__fma_rn(fabs(r), 1.0 + 0x1p-50, adel[i]) < h) & (at >= 0x1p-24) & (at < 0x1p30);
        ok[i] = tiny | inner;
        d0[i] = tiny ? 0.0 : t0;
    }
    double fl[4], rr[4];
    int idx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        fl[i] = floor(d0[i]);
        const double t16 = (d0[i] - fl[i]) * 65536.0;  // exact: d0 is an fp32 value below 2^30
        const double fi = floor(t16);
        idx[i] = (int)fi;
        rr[i] = t16 - fi;
    }
    double aa[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) aa[i] = T1s[idx[i] >> 8] * T2[idx[i] & 255];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const double poly = rr[i] * __fma_rn(rr[i], __fma_rn(rr[i], c3, c2), c1);
        const double Y = __fma_rn(aa[i], poly, aa[i]);
        const double Yr = (Y + 0x1.8p52) - 0x1.8p52;
        ok[i] = ok[i] & (fabs(Y - Yr) <= 0.5 - 0x1p-26);
        M[i] = (int)Yr;
        E[i] = (int)fl[i] - 23;
    }
}

// ------------------------------------------------------------------------------------------------
// Scores of 16 keys x 16 rows for one key group: straight-line MFMAs over the digit pairs (all 16
// when WIDE, else digits 1..3 of both: 9) into accumulators of equal weight s + t. kb[h]: this
// lane's K chunk base for dims 64 h + 16 g; qb[h]: its q chunk base (plane 0).
// ------------------------------------------------------------------------------------------------
template <bool WIDE>
__device__ __forceinline__ void score_mfma(const uint8_t* const (&kb)[2], const uint8_t* const (&qb)[2], int kt,
                                           v4i (&acc)[7]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        v4i Bq[4];
#pragma unroll
        for (int s = (WIDE ? 0 : 1); s < 4; ++s) Bq[s] = *(const v4i*)(qb[h] + 128 * s);
#pragma unroll
        for (int t = (WIDE ? 0 : 1); t < 4; ++t) {
            const v4i A = *(const v4i*)(kb[h] + t * 8192 + kt * 2048);
#pragma unroll
            for (int s = (WIDE ? 0 : 1); s < 4; ++s)
                acc[s + t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, Bq[s], acc[s + t], 0, 0, 0);
        }
    }
}

// fp64 value of sum_k acc_k 256^k for this lane's 4 keys, times 2^lk (units 2^lsbq). Adjacent
// accumulators combine exactly in int32 (|acc_k| <= 4 pairs x 2 x 64 x 2^14 = 2^23 for any k, and
// the pairs below reach 2^31 only with k >= 4 of at most 3 pairs: acc_k 256 + acc_(k-1) < 2^30.6 +
// 2^23); 3 fp64 roundings (the score bound allows 4). acc_0 = acc_1 = 0 for a narrow group.
__device__ __forceinline__ void score_fold(const v4i (&acc)[7], const v4i& lk, double (&xs)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int hi32 = acc[6][i] * 256 + acc[5][i];
        const int mid32 = acc[4][i] * 256 + acc[3][i];
        const int lo32 = acc[1][i] * 256 + acc[0][i];
        const double xx = __fma_rn(__fma_rn((double)hi32, 65536.0, (double)mid32), 256.0, (double)acc[2][i]);
        xs[i] = ldexp(__fma_rn(xx, 65536.0, (double)lo32), lk[i]);
    }
}


// s_waitcnt lgkmcnt(0) + s_barrier: LDS writes of every wave visible, outstanding DMAs untouched
__device__ __forceinline__ void pf_bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 16 bytes per lane from buffer rs at voff + soff into LDS at lds + 16 lane (M0 = lds, wave-
// uniform). The DMA counts in vmcnt; its consumers wait with wait_vm<n>. The compiler's hazard
// recognizer does not look inside inline asm: s_nop 4 gives the 5 wait states a VMEM read of an
// SGPR needs after a VALU write of it (v_readlane of a spilled soffset or descriptor word), which
// also covers the 1 wait state between an M0 write and an LDS DMA.
__device__ __forceinline__ void pf_dma(const v4i& rs, uint32_t lds, int voff, int soff) {
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rs), "s"(soff), "{m0}"(lds)
                 : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(const lds_void_t*)p);
}

}  // namespace pf
}  // namespace ea
