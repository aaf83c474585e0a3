// Certified prefill on the CDNA4 int8 matrix cores (gfx950): exact q.k scores and P.V sums from
// v_mfma_i32_16x16x64_i8 over balanced radix-256 digits of the bf16 inputs.
//
// Reference behaviour: the tensor-core split program of src/exactattn/triton_kernels.py
// (_tc_logits :395-482, _tc_pv :512-648, slices.slice_rows :31-52) and the definition in
// docs/SPEC.md. The arithmetic here is designed for CDNA4, not translated:
//
//   digits  a bf16 vector (q row, K row, V row) becomes integers X_i = x_i / 2^lsb with
//           |X_i| < 2^30, lsb = (top bit position over the vector) - 29, rounded to nearest where
//           an element lies more than 22 binades below the vector's top (counted, bounded).
//           X splits into 4 balanced digits d_s in [-128, 127], X = sum_s d_s 256^s: the bytes of
//           X + 0x80808080 with their top bits flipped. q and K use digits 1..3 (24 bits) unless
//           a digit 0 is nonzero (per wave of 16 rows, per 16-key group); V uses all four.
//   scores  S^T = K Q^T per 16 keys x 16 rows: one MFMA per digit pair and 64 dims, digit pairs of
//           equal weight s + t share an int32 accumulator (|acc| < 2^23). The fp64 Horner fold of
//           the 7 accumulators is within 6.01 u sum_i A_q,i A_k,i of the exact integer, and the
//           certified t = RN32(alpha s) is taken from that interval (ea_device.h logit_cert);
//           undecided pairs are recomputed exactly in the lane (TwoSum over bf16 products).
//   weights w = RN24(2^t) = M 2^E in fp64 (tables + cubic, 128-bit enclosure when undecided).
//   P.V     the S^T output layout leaves each lane 16 keys of one row, which is the A-operand
//           layout of the P.V MFMA (rows x keys): no transpose. Per row a base exponent; the
//           weight of key j enters as Wf = RN(M 2^(E + vlsb_j - base)) <= 2^38 (the V row's lsb
//           folded into the weight), as 5 balanced digits read straight out of the fp64 sum
//           Wf + 0x8080808080 + 1.5 * 2^52. acc_c = sum_j Wf_j X_jc over digit pairs s + t >= 2
//           (the 3 omitted pairs are bounded: 513 * 2^20 per tile), int32 accumulators kept
//           across tiles and folded into fp64 only when a row's base must move (a weight above
//           2^38) or after 256 tiles. Error bound per (row, channel):
//             |N/2^base - acc| <= sum_j |X_jc| / 2 + (2^38 + 1)/2 * (inexact V elements)
//                                 + omitted pairs + fold roundings.
//   Z       fp64 sum of the exact weights 2^(E - base), bound (n + 8) u' Z.
//   final   RN(N/Z) certified per channel (certify_round); rows with an undecided pair or
//           channel go to the device tier 2 work list, NaN/inf and logit overflow are flag 2.
//
// Kernels: ea_pf_qslice (q rows -> digits), ea_pf_kvslice (K/V pages -> 64-key digit tiles with
// per-key and per-channel metadata: the KV-cache slice format), ea_pf_main (one block of 4 waves
// per 64 rows of a segment, 16 rows per wave, K/V digit tiles DMA'd to LDS and double-buffered).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "ea_params.h"

using namespace ea;

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr double PF_U = 0x1p-53 * (1.0 + 0x1p-28);
// 1.5 * 2^52 + 0x8080808080: y = Wf + this has the biased digits of Wf in its low 40 bits
constexpr double PF_C40 = 6755399441055744.0 + (double)0x8080808080ull;

__device__ __forceinline__ void bf16_dec(uint32_t x, int* m, int* e, int* bad) {
    int f = (x >> 7) & 0xFF;
    int mm = (int)(x & 0x7F) | (f ? 0x80 : 0);
    *m = (x & 0x8000) ? -mm : mm;
    *e = (f ? f : 1) - 134;
    *bad = f == 0xFF;
}

__device__ __forceinline__ int lead_of(int m, int e) {
    int a = m < 0 ? -m : m;
    return e + 31 - __clz(a);
}

// X = RN(m 2^(e - lsb)) (half away from zero), with |m 2^(e - lsb)| < 2^30 guaranteed by lsb
__device__ __forceinline__ int to_fixed(int m, int e, int lsb, int* inexact) {
    int sh = e - lsb;
    int a = m < 0 ? -m : m;
    int r;
    if (sh >= 0) {
        r = a << sh;
        *inexact = 0;
    } else {
        int s = -sh;
        if (s > 10) {
            r = 0;
            *inexact = a != 0;
        } else {
            r = (a + (1 << (s - 1))) >> s;
            *inexact = (r << s) != a;
        }
    }
    return m < 0 ? -r : r;
}

// biased digit bytes of X (|X| < 2^30): byte s of the result, xor 0x80, is digit s
__device__ __forceinline__ uint32_t digits_u(int X) { return (uint32_t)X + 0x80808080u; }
__device__ __forceinline__ int digit(uint32_t u, int s) { return (int)(int8_t)(((u >> (8 * s)) & 0xFF) ^ 0x80); }
// sum_s |d_s| 256^s
__device__ __forceinline__ double digit_abs(uint32_t u) {
    double a = 0.0;
#pragma unroll
    for (int s = 3; s >= 0; --s) {
        int d = digit(u, s);
        a = a * 256.0 + (double)(d < 0 ? -d : d);
    }
    return a;
}

__device__ __forceinline__ double wave_max_d(double x) {
    for (int o = 32; o > 0; o >>= 1) x = fmax(x, __shfl_xor(x, o, 64));
    return x;
}

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
// Digits of 32 consecutive bf16 elements held by one lane; the 4 lanes of a quad (lane & 3) cover
// a 128-element vector. Returns the vector's lsb (quad-uniform) and fills X[32] and the digit
// bytes (4 planes x 32 bytes, as 8 dwords per plane).
// ------------------------------------------------------------------------------------------------
struct Slice32 {
    int lsb, bad, inex, need4, xmax;
    double amax, asum;
    uint32_t dig[4][8];
};

__device__ __forceinline__ int quad_max(int x) {
    x = max(x, __shfl_xor(x, 1, 64));
    return max(x, __shfl_xor(x, 2, 64));
}
__device__ __forceinline__ int quad_sum(int x) {
    x += __shfl_xor(x, 1, 64);
    return x + __shfl_xor(x, 2, 64);
}
__device__ __forceinline__ double quad_maxd(double x) {
    x = fmax(x, __shfl_xor(x, 1, 64));
    return fmax(x, __shfl_xor(x, 2, 64));
}
__device__ __forceinline__ double quad_sumd(double x) {
    x += __shfl_xor(x, 1, 64);
    return x + __shfl_xor(x, 2, 64);
}

// src: 32 bf16 values (any alignment of 2 bytes); valid = false gives an all-zero vector.
// lost[c] (optional) receives 1 for each element that is not exact in 30 bits.
__device__ __forceinline__ void slice32(const uint16_t* src, bool valid, Slice32& S, int* lost = nullptr) {
    int m[32], e[32];
    int bad = 0, lead = INT_MIN;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        int bk;
        bf16_dec(valid ? (uint32_t)src[k] : 0u, &m[k], &e[k], &bk);
        bad |= bk;
        if (m[k] && !bk) lead = max(lead, lead_of(m[k], e[k]));
    }
    lead = quad_max(lead);
    bad = quad_max(bad);
    const int lsb = (lead == INT_MIN) ? 0 : lead - 29;
    int inex = 0, need4 = 0, xmax = 0;
    double amax = 0.0, asum = 0.0;
#pragma unroll
    for (int w4 = 0; w4 < 8; ++w4) {
        uint32_t u[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int kk = 4 * w4 + k;
            int ie = 0;
            const int X = (bad || m[kk] == 0) ? 0 : to_fixed(m[kk], e[kk], lsb, &ie);
            inex += ie;
            if (lost) lost[kk] = ie;
            u[k] = digits_u(X);
            need4 |= digit(u[k], 0) != 0;
            const double a = digit_abs(u[k]);
            amax = fmax(amax, a);
            asum += a;
            xmax = max(xmax, X < 0 ? -X : X);
        }
        // plane s: byte k of dword w4 = digit s of element 4 w4 + k
#pragma unroll
        for (int sp = 0; sp < 4; ++sp) {
            uint32_t d = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) d |= (((u[k] >> (8 * sp)) & 0xFFu) ^ 0x80u) << (8 * k);
            S.dig[sp][w4] = d;
        }
    }
    S.lsb = lsb;
    S.bad = bad;
    S.inex = quad_sum(inex);
    S.need4 = quad_max(need4);
    S.xmax = quad_max(xmax);
    S.amax = quad_maxd(amax);
    S.asum = quad_sumd(asum);  // integers below 2^41: exact
}

}  // namespace

// ------------------------------------------------------------------------------------------------
// q rows -> digit planes: 64 rows per block, 4 lanes per row (32 dims each). Also clears the
// tier-2 work-list counter (this is the step's first kernel on the prefill path).
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) ea_pf_qslice(Params P) {
    if (blockIdx.x == 0 && threadIdx.x == 0) *P.wl_cnt = 0;
    const int q4 = threadIdx.x & 3;
    const int64_t row = (int64_t)blockIdx.x * 64 + (threadIdx.x >> 2);
    if (row >= P.rows) return;  // whole quads leave together
    const int Hq = P.g.num_q_heads, T = P.g.num_tokens;
    const int64_t b = row / ((int64_t)T * Hq);
    const int t = (int)((row / Hq) % T), hq = (int)(row % Hq);
    const uint16_t* qr = P.q + b * P.g.q_seq_stride + (int64_t)t * P.g.q_tok_stride + (int64_t)hq * P.g.q_head_stride;
    Slice32 S;
    slice32(qr + 32 * q4, true, S);
    uint8_t* dst = P.pfq + row * 512 + 32 * q4;
#pragma unroll
    for (int sp = 0; sp < 4; ++sp) {
        uint4* d4 = (uint4*)(dst + 128 * sp);
        d4[0] = make_uint4(S.dig[sp][0], S.dig[sp][1], S.dig[sp][2], S.dig[sp][3]);
        d4[1] = make_uint4(S.dig[sp][4], S.dig[sp][5], S.dig[sp][6], S.dig[sp][7]);
    }
    if (q4 == 0) {
        PfQMeta* qm = (PfQMeta*)P.pfqm + row;
        qm->lsb = S.lsb;
        qm->flags = S.need4 | (S.bad << 1) | (min(S.inex, 255) << 8);
        qm->qA = S.asum;
        qm->qX = (double)S.xmax;
        qm->a = ldexp(P.alpha, S.lsb);
    }
}

// ------------------------------------------------------------------------------------------------
// K/V pages -> one 64-key digit tile per block (segment-major), in the LDS layout of ea_pf_main.
// Lane quad (key = tid / 4) covers the key's 128 dims and 128 channels. K planes are written
// straight to memory in 16-byte chunks; the V planes (keys interleaved per channel) are
// assembled in LDS and copied out in 16-byte chunks.
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) ea_pf_kvslice(Params P) {
    __shared__ __align__(16) uint8_t s_v[32768];
    __shared__ int s_lc[128];
    __shared__ int s_tfl;
    const int tid = threadIdx.x, q4 = tid & 3, key = tid >> 2;
    const int seg = blockIdx.x / P.pf_ntiles, tile = blockIdx.x % P.pf_ntiles;
    const int Hkv = P.g.num_kv_heads;
    const int64_t b = seg / Hkv;
    const int hk = seg % Hkv;
    uint8_t* T = P.pfkv + ((int64_t)seg * P.pf_ntiles + tile) * EA_PF_TILE_BYTES;
    PfTileMeta* TM = (PfTileMeta*)(T + EA_PF_META_OFF);
    if (tid < 128) s_lc[tid] = 0;
    if (tid == 0) s_tfl = 0;
    __syncthreads();
    const int64_t n = (int64_t)tile * 64 + key;
    const bool valid = n < P.seq_len[b];
    const uint16_t* kr = P.k + (valid ? kv_off(P, b, n, hk, 0) : 0) + 32 * q4;
    const uint16_t* vr = P.v + (valid ? kv_off(P, b, n, hk, 1) : 0) + 32 * q4;
    int bad;
    {
        Slice32 S;
        slice32(kr, valid, S);
#pragma unroll
        for (int sp = 0; sp < 4; ++sp) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int c = 2 * q4 + hh;  // 16-byte chunk of dims 16c .. 16c+15
                *(uint4*)(T + sp * 8192 + key * 128 + ((c ^ (key & 7)) << 4)) =
                    make_uint4(S.dig[sp][4 * hh], S.dig[sp][4 * hh + 1], S.dig[sp][4 * hh + 2], S.dig[sp][4 * hh + 3]);
            }
        }
        bad = S.bad;
        if (q4 == 0) {
            TM->lsbk[key] = S.lsb;
            TM->kA[key] = S.amax;
            TM->kX[key] = (double)S.xmax;
        }
        int tf = (S.need4 ? 1 : 0) << (key >> 4);
        if (S.inex) tf |= 32;
        if (q4 == 0 && tf) atomicOr(&s_tfl, tf);
        bad |= 0;
        if (q4 == 0) TM->kfl[key] = min(S.inex, 255) << 8;  // bit 0 set below with V
    }
    {
        Slice32 S;
        int lost[32];
        slice32(vr, valid, S, lost);
        const int gq = (key >> 2) & 3, kt = key >> 4, ii = key & 3;
#pragma unroll
        for (int sp = 0; sp < 4; ++sp)
#pragma unroll
            for (int k = 0; k < 32; ++k) {
                const int ch = 32 * q4 + k;
                s_v[sp * 8192 + ch * 64 + ((gq ^ ((ch >> 1) & 3)) << 4) + 4 * kt + ii] =
                    (uint8_t)(S.dig[sp][k >> 2] >> (8 * (k & 3)));
            }
        if (S.inex) {
#pragma unroll
            for (int k = 0; k < 32; ++k)
                if (lost[k]) atomicAdd(&s_lc[32 * q4 + k], 1);
        }
        bad = quad_max(bad | S.bad);
        if (q4 == 0) {
            TM->vlsb[key] = S.lsb;
            if (bad) {
                TM->kfl[key] |= 1;
                atomicOr(&s_tfl, 16);
            }
        }
    }
    __syncthreads();
    const uint4* sv4 = (const uint4*)s_v;
    uint4* dv4 = (uint4*)(T + 32768);
#pragma unroll
    for (int i = 0; i < 8; ++i) dv4[tid + 256 * i] = sv4[tid + 256 * i];
    if (tid < 128) TM->EV[tid] = 0.5 * (0x1p38 + 1.0) * (double)s_lc[tid];
    if (tid == 0) {
        int tot = 0;
        for (int c = 0; c < 128; ++c) tot += s_lc[c];
        TM->tfl = s_tfl;
        TM->EVt = 0.5 * (0x1p38 + 1.0) * (double)tot;
    }
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
// Branch-free certified t = RN32(alpha s) and w = RN24(2^t) = M 2^E for 4 pairs in lock step
// (independent chains the scheduler interleaves). x: fp64 scores in units 2^(lsbq + lk), within
// adx / |a| of the exact integers; a = alpha 2^lsbq. The interval around a x 2^lk rounds to
// t0 = RN32(p) when it lies inside the smaller half gap next to t0: 2^(e - 24) for |t0| in
// [2^e, 2^(e+1)), 2^(e - 25) when |t0| is a power of two (the gap below it is half as wide);
// |alpha s| <= 2^-25 gives w = 1. 2^f from the fp64 tables (T1 pre-scaled by 2^23) and the
// cubic, rounded to an integer by adding and subtracting 1.5 * 2^52; certified when
// |Y - RN(Y)| <= 1/2 - 2^-26 (the fp64 evaluation error is below 2^-26.9). ok[i] false: the exact
// path decides.
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ void lean_weight4(const double (&x)[4], const double (&adx)[4], const v4i& lk, double a,
                                             const double* T1s, const double* T2, int (&M)[4], int (&E)[4],
                                             bool (&ok)[4]) {
    const double c1 = u64_as_f64(EA_C_BITS[0]), c2 = u64_as_f64(EA_C_BITS[1]), c3 = u64_as_f64(EA_C_BITS[2]);
    double p[4], pe[4], d0[4], adel[4];
    int idx[4];
    double f[4], fl[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const double xs = ldexp(x[i], lk[i]);
        adel[i] = ldexp(adx[i], lk[i]) * (1.0 + 0x1p-50);
        p[i] = a * xs;
        pe[i] = __fma_rn(a, xs, -p[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float tf = (float)p[i];
        const double t0 = (double)tf;
        const double r = (p[i] - t0) + pe[i];
        const uint32_t hx = (uint32_t)__double2hiint(t0) & 0x7FF00000u;
        const uint32_t hsh = (__float_as_uint(tf) & 0x7FFFFFu) ? (24u << 20) : (25u << 20);
        const double h = __hiloint2double((int)(hx - hsh), 0);
        const bool tiny = fabs(p[i]) + fabs(pe[i]) + adel[i] <= 0x1p-25 * (1.0 - 0x1p-20);
        const double at = fabs(t0);
        const bool inner = (fabs(r) * (1.0 + 0x1p-52) + adel[i] + 0x1p-1060 < h) & (at >= 0x1p-24) & (at < 0x1p30);
        ok[i] = tiny | inner;
        d0[i] = tiny ? 0.0 : t0;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        fl[i] = floor(d0[i]);
        f[i] = d0[i] - fl[i];
        idx[i] = ((int)(f[i] * 65536.0)) & 0xFFFF;
    }
    double aa[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) aa[i] = T1s[idx[i] >> 8] * T2[idx[i] & 255];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const double rr = __fma_rn(-(double)idx[i], 0x1p-16, f[i]);
        const double poly = rr * __fma_rn(rr, __fma_rn(rr, c3, c2), c1);
        const double Y = __fma_rn(aa[i], poly, aa[i]);
        const double Yr = (Y + 0x1.8p52) - 0x1.8p52;
        ok[i] = ok[i] & (fabs(Y - Yr) <= 0.5 - 0x1p-26);
        M[i] = (int)Yr;
        E[i] = (int)fl[i] - 23;
    }
}

// ------------------------------------------------------------------------------------------------
// Scores of 16 keys x 16 rows for one key group: straight-line MFMAs over the digit pairs (all 16
// when WIDE, else digits 1..3 of both: 9) into accumulators of equal weight, then the fp64 value of
// sum_k acc_k 256^k for this lane's 4 keys. Adjacent accumulators combine exactly in int32
// (|acc_k| <= 4 pairs x 2 x 64 x 2^14 = 2^23 for any k, and the pairs below reach 2^31 only with
// k >= 4 of at most 3 pairs: acc_k 256 + acc_(k-1) < 2^30.6 + 2^23); at most 4 fp64 roundings.
// kb[h]: this lane's K chunk base for dims 64 h + 16 g; qb[h]: its q chunk base (plane 0).
// ------------------------------------------------------------------------------------------------
template <bool WIDE>
__device__ __forceinline__ void score_group(const uint8_t* const (&kb)[2], const uint8_t* const (&qb)[2], int kt,
                                            double (&x)[4]) {
    v4i acc[7];
#pragma unroll
    for (int k = 0; k < 7; ++k) acc[k] = (v4i){0, 0, 0, 0};
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
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int hi32 = acc[6][i] * 256 + acc[5][i];
        const int mid32 = acc[4][i] * 256 + acc[3][i];
        double xx = __fma_rn(__fma_rn((double)hi32, 65536.0, (double)mid32), 256.0, (double)acc[2][i]);
        if (WIDE) xx = __fma_rn(xx, 65536.0, (double)(acc[1][i] * 256 + acc[0][i]));
        else xx *= 65536.0;
        x[i] = xx;
    }
}

// ------------------------------------------------------------------------------------------------
// Main kernel. Block = 8 waves over 64 consecutive rows (tokens x query heads of one KV head).
// Waves 2 rg and 2 rg + 1 share the 16 rows of row group rg; wave half hh = w & 1 takes the
// scores and weights of key groups kt = 2 hh, 2 hh + 1 of each tile and the P.V sums of channel
// tiles ct = 4 hh .. 4 hh + 3. The pair exchanges row maxima and weight digits through LDS.
// Lane (g = lane / 16, j = lane % 16):
//   score layout  row j, keys 16 kt + 4 g + i (i = 0..3)
//   P.V layout    rows 4 g + i, channels 16 ct + j
// LDS: K and V planes single-buffered (the next tile's K planes load during this tile's weight
// and P.V phases, its V planes during the next score phase), tile metadata double-buffered, the
// block's q digits, exp2 tables, the pair exchanges.
// ------------------------------------------------------------------------------------------------
constexpr int PF_OFF_V = 0;                      // V planes (32 KB), single buffer
constexpr int PF_OFF_K = 32768;                  // K planes (32 KB), single buffer
constexpr int PF_OFF_M = 65536;                  // tile metadata, 2 x 4 KB
constexpr int PF_OFF_Q = PF_OFF_M + 8192;        // q digits of the block's 64 rows (32 KB)
constexpr int PF_OFF_T = PF_OFF_Q + 32768;       // T1 * 2^23, T2 (4 KB)
constexpr int PF_OFF_WD = PF_OFF_T + 4096;       // weight digits: 8 waves x 5 planes x 2 x 64 lanes
constexpr int PF_OFF_X = PF_OFF_WD + 8 * 2560;   // per-lane exchange: 8 waves x 64 lanes x 16 B
constexpr int PF_LDS = PF_OFF_X + 8 * 1024;

struct PfX {
    int32_t a, b;
    double c;
};

template <int SPLIT, int NWB, bool TIMERS>
__global__ void __launch_bounds__(64 * NWB, 1) ea_pf_main(Params P) {
    // phase clocks (TIMERS build): shader cycles summed over waves into P.timers[0..7]:
    // [0] wait for K + barrier, [1] scores and weights, [2] pair exchange, [3] epoch folds,
    // [4] weight digits, [5] wait for V + barrier, [6] P.V, [7] barrier after P.V
    uint64_t tclk[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint64_t tprev = TIMERS ? __builtin_amdgcn_s_memtime() : 0;
    auto tick = [&](int ph) __attribute__((always_inline)) {
        if (TIMERS) {
            const uint64_t t = __builtin_amdgcn_s_memtime();
            tclk[ph] += t - tprev;
            tprev = t;
        }
    };
    constexpr int RPB = 16 * NWB / SPLIT;  // rows per block
    constexpr int NKT = 4 / SPLIT;     // key groups of 16 per wave
    constexpr int NCT = 8 / SPLIT;     // channel tiles of 16 per wave
    constexpr int NKI = 32 / NWB;      // K (and V) DMA instructions per wave and tile
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int s_kend;
    double* const T1s = (double*)(smem + PF_OFF_T);
    double* const T2 = T1s + 256;
    uint32_t* const s_wd = (uint32_t*)(smem + PF_OFF_WD);  // [wave][plane 5][2][lane 64]
    PfX* const s_x = (PfX*)(smem + PF_OFF_X);              // [wave][lane 64]
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = w / SPLIT, hh = w % SPLIT;
    const int g = lane >> 4, j = lane & 15;
    const int nseg = P.nseg;
    const int seg = blockIdx.x % nseg;
    const int rbk = P.pf_nrb - 1 - (int)(blockIdx.x / nseg);
    const int Hkv = P.g.num_kv_heads;
    const int64_t b = seg / Hkv;
    const int hk = seg % Hkv;
    const int T = P.g.num_tokens;
    uint32_t* const wd_w = s_wd + w * 640 + lane;               // this wave's digit planes (SPLIT 2)
    const uint32_t* const wd_r = s_wd + (w & ~1) * 640 + lane;  // the pair's, in key-group order
    // per-lane scratch: fp64 sums of completed epochs, then the final quotients
    double* const scr = P.pfscr + (((int64_t)blockIdx.x * NWB + w) * 64 + lane) * (8 * NCT);

    if (tid == 0) s_kend = 0;
    if (tid < 256) {
        T1s[tid] = u64_as_f64(EA_T1_BITS[tid]) * 8388608.0;  // 2^23: exact
        T2[tid] = u64_as_f64(EA_T2_BITS[tid]);
    }
    // ---- this lane's row in the score layout
    const int lr = rbk * RPB + rg * 16 + j;
    const bool rvalid = lr < P.r_seg;
    const int lrc = rvalid ? lr : P.r_seg - 1;
    int tq;
    const int64_t grow = seg_row(P, b, hk, lrc, &tq);
    const int64_t tok = b * T + tq;
    const int kvl = rvalid ? P.kv_len[tok] : 0;
    const uint64_t tmk = (rvalid && P.tree_mask) ? P.tree_mask[tok] : 0ull;
    const int tbase = P.tree_mask ? P.tree_base[b] : 0;
    const int slen = P.seq_len[b];
    int ve = kvl;
    if (tmk) ve = max(ve, tbase + 64 - (int)__clzll(tmk));
    ve = min(ve, slen);
    __syncthreads();  // s_kend initialised
    {
        const int kw = wave_max_i(ve);
        if (lane == 0) atomicMax(&s_kend, kw);
    }
    // q digits of the block's rows into LDS: [row][plane 4][128 bytes], 16-byte chunk c of row r
    // at chunk c ^ (r & 7) (conflict-free reads across the 8 rows of a lane group); rows past the
    // segment repeat its last row
    for (int c = tid; c < RPB * 32; c += 64 * NWB) {
        const int r = c >> 5, q16 = c & 31;
        const int lrr = min(rbk * RPB + r, P.r_seg - 1);
        int tt;
        const int64_t gr = seg_row(P, b, hk, lrr, &tt);
        *(uint4*)(smem + PF_OFF_Q + r * 512 + ((q16 ^ (r & 7)) << 4)) = *(const uint4*)(P.pfq + gr * 512 + q16 * 16);
    }
    // this lane's q digits (B operand of the score MFMA): row j, dims 64 h + 16 g .. + 15, plane s:
    // chunk 8 s + 4 h + g of the row, swizzled
    const uint8_t* const qlds = smem + PF_OFF_Q + (rg * 16 + j) * 512;
    // (8 s + 4 h + g) ^ (j & 7) = 8 s + ((4 h + g) ^ (j & 7)): one base per h, plane s at + 128 s
    const uint8_t* const qb[2] = {qlds + ((g ^ (j & 7)) << 4), qlds + (((4 + g) ^ (j & 7)) << 4)};
    // K operand: key 16 kt + j, chunk (4 h + g) ^ (j & 7), plane t at + 8192 t, key group at + 2048 kt
    const uint8_t* const kb[2] = {smem + PF_OFF_K + j * 128 + ((g ^ (j & 7)) << 4),
                                  smem + PF_OFF_K + j * 128 + (((4 + g) ^ (j & 7)) << 4)};
    const PfQMeta qm = ((const PfQMeta*)P.pfqm)[grow];
    const bool needq = __ballot(rvalid && (qm.flags & 1)) != 0;
    // |a| times the fold error factor 6.01 u and sum_i A_q,i: the score bound is this * A_k
    const double adq = fabs(qm.a) * 6.01 * 0x1p-53 * qm.qA;
    const double aqL = fabs(qm.a) * 0.5 * (double)((qm.flags >> 8) & 0xFF);
    const double aqX = fabs(qm.a) * 0.5 * (qm.qX + 1.0);
    const bool lossy_q = __ballot(rvalid && ((qm.flags >> 8) & 0xFF)) != 0;
    const bool qbad = (qm.flags & 2) != 0;
    int dom = (rvalid && qbad) ? 1 : 0;  // NaN/inf in q: a domain error (docs/SPEC.md)
    int unc = 0;
    int nslow = 0, nunc_s = 0, nunc_w = 0;
    __syncthreads();  // s_kend final, tables visible
    const int kend = s_kend;
    const int ntiles = (kend + 63) >> 6;

    // tile DMA: K planes and metadata into K buffer `buf`, V planes into the V buffer. Per wave:
    // 4 K instructions (+1 metadata for waves 0..3), 4 V instructions.
    auto rsrc = [&](int tile) __attribute__((always_inline)) {
        const uint8_t* src = P.pfkv + ((int64_t)seg * P.pf_ntiles + tile) * EA_PF_TILE_BYTES;
        return __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, EA_PF_TILE_BYTES, 0x00020000);
    };
    // one lane offset for every DMA instruction; the per-instruction offset goes in soffset
    const int vlane = lane * 16;
    auto issue_k = [&](int tile) __attribute__((always_inline)) {
        __amdgpu_buffer_rsrc_t rs = rsrc(tile);
#pragma unroll
        for (int q = 0; q < NKI; ++q) {
            const int off = (q * NWB + w) * 1024;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(smem + PF_OFF_K + off), 16, vlane, off, 0, 0);
        }
        if (NWB == 4 || w < 4)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(smem + PF_OFF_M + (tile & 1) * 4096 + w * 1024),
                                                     16, vlane, EA_PF_META_OFF + w * 1024, 0, 0);
    };
    auto issue_v = [&](int tile) __attribute__((always_inline)) {
        __amdgpu_buffer_rsrc_t rs = rsrc(tile);
#pragma unroll
        for (int q = 0; q < NKI; ++q) {
            const int off = (q * NWB + w) * 1024;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(smem + PF_OFF_V + off), 16, vlane, 32768 + off,
                                                     0, 0);
        }
    };

    // per-row state (score layout; the 4 lanes of a row, and both waves of the pair, hold the
    // same base)
    int base = INT_MIN;
    double z = 0.0;  // this wave's keys
    int nv = 0;
    int nfrac = 0;   // this wave's keys of the current epoch whose scaled weight may have a fraction
    // P.V state (P.V layout): int32 accumulators of digit weights 256^1 .. 256^7, 4 channel tiles
    v4i pacc[NCT][7];
#pragma unroll
    for (int cc = 0; cc < NCT; ++cc)
#pragma unroll
        for (int k = 0; k < 7; ++k) pacc[cc][k] = (v4i){0, 0, 0, 0};
    double EVs[NCT];  // per channel: inexact V elements of the epoch's tiles, times (2^38 + 1) / 2
#pragma unroll
    for (int cc = 0; cc < NCT; ++cc) EVs[cc] = 0.0;
    int ep_tiles = 0;
    bool had_fold = false;  // scr holds the sums of earlier epochs
    uint32_t failbits = 0;

    if (ntiles > 0) {
        issue_k(0);
        issue_v(0);
    }
    for (int it = 0; it <= ntiles; ++it) {
        const bool last = it == ntiles;
        const uint8_t* Kt = smem + PF_OFF_K;
        const PfTileMeta* TM = (const PfTileMeta*)(smem + PF_OFF_M + (it & 1) * 4096);
        v4i Mk[NKT], Ek[NKT];
        int nb = base;
        bool do_fold;
        int nf_pair = 0;  // the pair's nfrac (epoch so far)
        bool k_next = false;
        if (!last) {
            tick(7);
            wait_vm<NKI>();   // K(it) and its metadata landed; V(it) (NKI instructions) may be in flight
            __syncthreads();  // for every wave
            tick(0);
            k_next = it + 1 < ntiles;
            const int tfl = TM->tfl;
            const bool lossy = lossy_q || (tfl & 32);
            uint32_t slowmask = 0;  // pairs the fast path left undecided (cold path below)
            int gm = INT_MIN;
#pragma unroll
            for (int kk = 0; kk < NKT; ++kk) {
                const int kt = NKT * hh + kk;
                const bool wide = needq || ((tfl >> kt) & 1);
                double x[4];
                if (wide) score_group<true>(kb, qb, kt, x);
                else score_group<false>(kb, qb, kt, x);
                const v4i lsbk4 = *(const v4i*)&TM->lsbk[16 * kt + 4 * g];
                const v4i kfl4 = *(const v4i*)&TM->kfl[16 * kt + 4 * g];
                const v4i vl4 = *(const v4i*)&TM->vlsb[16 * kt + 4 * g];
                const double2 kA01 = *(const double2*)&TM->kA[16 * kt + 4 * g];
                const double2 kA23 = *(const double2*)&TM->kA[16 * kt + 4 * g + 2];
                const double kA[4] = {kA01.x, kA01.y, kA23.x, kA23.y};
                double adx[4];
                bool vis[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int n = it * 64 + 16 * kt + 4 * g + i;
                    const int ti = n - tbase;
                    const bool intree = ((unsigned)ti < 64u) & (((tmk >> (ti & 63)) & 1ull) != 0);
                    vis[i] = (n < slen) & ((n < kvl) | intree);
                    adx[i] = adq * kA[i];
                }
                if (lossy) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        adx[i] = __fma_rn(aqL, TM->kX[16 * kt + 4 * g + i] + 1.0, __fma_rn((double)(kfl4[i] >> 8), aqX, adx[i]));
                }
                int M[4], E[4];
                bool ok[4];
                lean_weight4(x, adx, lsbk4, qm.a, T1s, T2, M, E, ok);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool kbad = kfl4[i] & 1;
                    const bool good = vis[i] & ok[i] & !kbad;
                    dom |= (vis[i] & kbad) ? 1 : 0;
                    slowmask |= (vis[i] & !ok[i] & !kbad) ? (1u << (4 * kk + i)) : 0u;
                    Mk[kk][i] = good ? M[i] : 0;
                    Ek[kk][i] = E[i];
                    gm = max(gm, good ? E[i] + vl4[i] : INT_MIN);
                }
            }
            // ---- cold path: exact decision for the pairs the fast path left undecided. The exact
            // integer score comes from the digit planes in LDS (no memory traffic); only pairs
            // whose digits are inexact (elements rounded at slicing) read the bf16 inputs.
            if (__builtin_expect(__ballot(slowmask != 0) != 0, 0)) {
                if (P.stats && lane == 0) atomicAdd((unsigned long long*)&P.stats[12], 1ull);
                for (int p = 0; p < 4 * NKT; ++p) {
                    if (!((slowmask >> p) & 1)) continue;
                    const int kk = p >> 2, i = p & 3;
                    const int key = 16 * (NKT * hh + kk) + 4 * g + i;
                    const int n = it * 64 + key;
                    const int kf = TM->kfl[key];
                    uint32_t tbits = 0;
                    int ls = 3;
                    ++nslow;
                    if (!qbad && !((qm.flags >> 8) & 0xFF) && !(kf >> 8)) {
                        const int8_t* qrow = (const int8_t*)qlds;
                        const int8_t* krow = (const int8_t*)(Kt + key * 128);
                        i128 S = 0;
                        for (int c = 0; c < 128; ++c) {
                            const int kc = (((c >> 4) ^ (key & 7)) << 4) | (c & 15);
                            int xq = 0, xk = 0;
#pragma unroll
                            for (int sp = 3; sp >= 0; --sp) {
                                xq = xq * 256 + (int)qrow[(((8 * sp + (c >> 4)) ^ (j & 7)) << 4) | (c & 15)];
                                xk = xk * 256 + (int)krow[8192 * sp + kc];
                            }
                            S += (i128)((int64_t)xq * (int64_t)xk);
                        }
                        ls = rn32_prod(P.am, S, P.ae + qm.lsb + TM->lsbk[key], &tbits);
                    } else if (!qbad) {
                        const uint16_t* qr = P.q + b * P.g.q_seq_stride + (int64_t)tq * P.g.q_tok_stride +
                                             (int64_t)(hk * P.grp + lrc % P.grp) * P.g.q_head_stride;
                        const uint16_t* kr = P.k + kv_off(P, b, n, hk, 0);
                        double ss = 0.0, es = 0.0, ea = 0.0;
                        for (int c = 0; c < 128; ++c) {
                            double e0;
                            ss = two_sum(ss, (double)__uint_as_float((uint32_t)qr[c] << 16) *
                                                 (double)__uint_as_float((uint32_t)kr[c] << 16), &e0);
                            es += e0;
                            ea += fabs(e0);
                        }
                        ls = (ss == 0.0 && es == 0.0 && ea == 0.0) ? 1
                                                                    : logit_cert(P.alpha, ss, es, ea * 0x1p-44, &tbits);
                        if (ls == 1) tbits = 0;
                    }
                    int32_t M = 0, E = 0;
                    bool live = false;
                    if (ls == 2) {
                        dom = 1;
                    } else if (ls == 3) {
                        unc = 1;
                        ++nunc_s;
                    } else if (table_weight(tbits, T1s, T2, &M, &E)) {
                        live = true;
                    } else {
                        // the 128-bit enclosure of 2^t decides RN24 (ea_device.h weight_wide)
                        int32_t M2 = 0;
                        int64_t E2 = 0;
                        if (weight_wide(tbits, &M2, &E2) == 0 && E2 > -(1LL << 30) && E2 < (1LL << 30)) {
                            M = M2;
                            E = (int32_t)E2;
                            live = true;
                        } else {
                            unc = 1;
                            ++nunc_w;
                        }
                    }
#pragma unroll
                    for (int q = 0; q < NKT; ++q)
                        if (q == kk) {
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                if (r == i) {
                                    Mk[q][r] = live ? M : 0;
                                    Ek[q][r] = E;
                                }
                        }
                    if (live) gm = max(gm, E + TM->vlsb[key]);
                }
            }
            // ---- the row's largest weight in this tile (both waves of the pair); the base moves
            // when a weight would exceed 2^38 (G - base > 14 for G = E + vlsb)
            gm = max(gm, __shfl_xor(gm, 16, 64));
            gm = max(gm, __shfl_xor(gm, 32, 64));
            tick(1);
            if (SPLIT == 2) s_x[w * 64 + lane] = PfX{gm, nfrac, 0.0};
            __syncthreads();  // every wave is done with the K planes of tile it
            if (k_next) issue_k(it + 1);
            nf_pair = nfrac;
            if (SPLIT == 2) {
                const PfX o = s_x[(w ^ 1) * 64 + lane];
                gm = max(gm, o.a);
                nf_pair += o.b;
            }
            const bool need_rb = gm != INT_MIN && (base == INT_MIN || gm > base + 14);
            nb = need_rb ? gm - 10 : base;
            do_fold = ep_tiles > 0 && (__ballot(need_rb) != 0 || ep_tiles >= 256);
            tick(2);
        } else {
            // row totals for the final rounding: this wave's 4 lanes of the row, then the partner
            z += __shfl_xor(z, 16, 64);
            z += __shfl_xor(z, 32, 64);
            nv += __shfl_xor(nv, 16, 64);
            nv += __shfl_xor(nv, 32, 64);
            dom |= __shfl_xor(dom, 16, 64);
            dom |= __shfl_xor(dom, 32, 64);
            unc |= __shfl_xor(unc, 16, 64);
            unc |= __shfl_xor(unc, 32, 64);
            nf_pair = nfrac;
            if (SPLIT == 2) {
                s_x[w * 64 + lane] = PfX{nv, nfrac | (dom << 24) | (unc << 25), z};
                __syncthreads();
                const PfX o = s_x[(w ^ 1) * 64 + lane];
                nv += o.a;
                nf_pair += o.b & 0xFFFFFF;
                dom |= (o.b >> 24) & 1;
                unc |= (o.b >> 25) & 1;
                z += o.c;
            }
            do_fold = true;
        }
        if (do_fold) {
            if (P.stats && lane == 0 && !last) atomicAdd((unsigned long long*)&P.stats[11], 1ull);
            // fold the int32 P.V accumulators (units 2^base of each row) into fp64 with a bound.
            // Before the last tile: add into scr, rescaled to the new bases. At the end: the
            // quotient N/Z and its error radius per (row, channel), certified further below.
            int nf = nf_pair + __shfl_xor(nf_pair, 16, 64);
            nf += __shfl_xor(nf, 32, 64);
            double Zs[4], eZs[4], fr[4];
            bool live_i[4];
            int bo[4], bn[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                bo[i] = __shfl(base, 4 * g + i, 64);
                bn[i] = __shfl(nb, 4 * g + i, 64);
                fr[i] = 0x1p29 * (double)__shfl(nf, 4 * g + i, 64);  // weight roundings: 2^30 / 2 each
                Zs[i] = eZs[i] = 0.0;
                live_i[i] = false;
                if (last) {
                    Zs[i] = __shfl(z, 4 * g + i, 64);
                    const int nvr = __shfl(nv, 4 * g + i, 64);
                    eZs[i] = (double)(nvr + 8) * PF_U * Zs[i] + (double)(nvr + 64) * 0x1p-1074;
                    live_i[i] = nvr > 0 && !__shfl(dom | unc, 4 * g + i, 64);
                }
            }
            nfrac = 0;
            const double omit = (double)ep_tiles * 0x1p20;  // pair (0, 0): 64 keys x 2^14
#pragma unroll
            for (int cc = 0; cc < NCT; ++cc) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    double h = (double)pacc[cc][6][i], ha = fabs(h);
#pragma unroll
                    for (int k = 5; k >= 0; --k) {
                        const double a = (double)pacc[cc][k][i];
                        h = __fma_rn(h, 256.0, a);
                        ha = __fma_rn(ha, 256.0, fabs(a));
                    }
                    h *= 256.0;
                    ha *= 256.0;
                    double en = 6.02 * 0x1p-53 * ha + EVs[cc] + omit + fr[i];
                    double nn = h;
                    double2* sp = (double2*)(scr + 2 * (4 * cc + i));
                    if (had_fold) {
                        const double2 o = *sp;
                        nn += o.x;
                        en += o.y;
                    }
                    en += fabs(nn) * 0x1p-52;
                    if (!last) {
                        if (bo[i] != INT_MIN && bn[i] != bo[i]) {
                            const int dsh = max(bo[i] - bn[i], -1100);
                            nn = ldexp(nn, dsh);
                            en = ldexp(en, dsh) + 0x1p-1074;
                        }
                        *sp = make_double2(nn, en);
                    } else {
                        double q = 0.0, delta = -1.0;  // delta < 0: no output from this entry
                        const double Z = Zs[i], eZ = eZs[i];
                        if (live_i[i]) {
                            if (Z > 2.0 * eZ && isfinite(Z)) {
                                q = nn / Z;
                                delta = (en * (1.0 + 0x1p-40) + fabs(q) * eZ) / (Z - eZ) * (1.0 + 0x1p-40) +
                                        fabs(q) * 0x1p-51 + 0x1p-1070;
                                if (!isfinite(q) || !isfinite(delta)) delta = __builtin_inf();
                            } else {
                                delta = __builtin_inf();
                            }
                        }
                        *sp = make_double2(q, delta);
                    }
#pragma unroll
                    for (int k = 0; k < 7; ++k) pacc[cc][k][i] = 0;
                }
            }
#pragma unroll
            for (int cc = 0; cc < NCT; ++cc) EVs[cc] = 0.0;
            ep_tiles = 0;
            had_fold = !last;
            wait_vm<0>();  // the scr stores are complete (keeps the DMA counts below exact)
            tick(3);
        }
        if (last) break;
        // ---- move bases, then this wave's weight digits (A operand of the P.V MFMA) and Z
        if (nb != base && base != INT_MIN) z = ldexp(z, max(base - nb, -1100));
        base = nb;
        v4i Wd[5];
#pragma unroll
        for (int kk = 0; kk < NKT; ++kk) {
            const int kt = NKT * hh + kk;
            uint32_t L[4], H[4];
            const v4i vl4 = *(const v4i*)&TM->vlsb[16 * kt + 4 * g];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int Mp = Mk[kk][i];
                const int sc = Ek[kk][i] - base;
                const double md = (double)Mp;
                const double wsc = ldexp(md, sc + vl4[i]);  // <= 2^38
                z += ldexp(md, sc);                         // md = 0 for masked pairs
                nv += Mp ? 1 : 0;
                nfrac += (Mp && sc + vl4[i] < 0) ? 1 : 0;
                const uint64_t yb = f64_as_u64(wsc + PF_C40);
                L[i] = (uint32_t)yb;
                H[i] = (uint32_t)(yb >> 32);
            }
            const uint32_t a01 = __builtin_amdgcn_perm(L[1], L[0], 0x05010400u);
            const uint32_t b01 = __builtin_amdgcn_perm(L[1], L[0], 0x07030602u);
            const uint32_t a23 = __builtin_amdgcn_perm(L[3], L[2], 0x05010400u);
            const uint32_t b23 = __builtin_amdgcn_perm(L[3], L[2], 0x07030602u);
            const uint32_t e01 = __builtin_amdgcn_perm(H[1], H[0], 0x05010400u);
            const uint32_t e23 = __builtin_amdgcn_perm(H[3], H[2], 0x05010400u);
            const uint32_t d0 = __builtin_amdgcn_perm(a23, a01, 0x05040100u) ^ 0x80808080u;
            const uint32_t d1 = __builtin_amdgcn_perm(a23, a01, 0x07060302u) ^ 0x80808080u;
            const uint32_t d2 = __builtin_amdgcn_perm(b23, b01, 0x05040100u) ^ 0x80808080u;
            const uint32_t d3 = __builtin_amdgcn_perm(b23, b01, 0x07060302u) ^ 0x80808080u;
            const uint32_t d4 = __builtin_amdgcn_perm(e23, e01, 0x05040100u) ^ 0x80808080u;
            if (SPLIT == 2) {
                uint32_t* wd = wd_w + kk * 64;
                wd[0 * 128] = d0;
                wd[1 * 128] = d1;
                wd[2 * 128] = d2;
                wd[3 * 128] = d3;
                wd[4 * 128] = d4;
            } else {
                Wd[0][kt] = (int)d0;
                Wd[1][kt] = (int)d1;
                Wd[2][kt] = (int)d2;
                Wd[3][kt] = (int)d3;
                Wd[4][kt] = (int)d4;
            }
        }
        tick(4);
        // V(it) landed (only K(it+1) may still be in flight), the pair's digits are in LDS
        if (k_next) {
            if (NWB == 4 || w < 4) wait_vm<NKI + 1>();
            else wait_vm<NKI>();
        } else {
            wait_vm<0>();
        }
        __syncthreads();
        tick(5);
        if (SPLIT == 2) {
#pragma unroll
            for (int s = 0; s < 5; ++s)
#pragma unroll
                for (int kt = 0; kt < 4; ++kt) Wd[s][kt] = (int)wd_r[(kt >> 1) * 640 + (s * 2 + (kt & 1)) * 64];
        }
        // ---- P.V: pacc[cc][s + t - 1] += W digits s x V digits t (all pairs but (0, 0))
        // channel 16 (NCT hh + cc) + j: the 16-byte slot swizzle (ch >> 1) & 3 = (j >> 1) & 3 does
        // not depend on cc, so every read is one lane base plus a constant
        const uint8_t* Vt = smem + PF_OFF_V + (16 * NCT * hh + j) * 64 + ((g ^ ((j >> 1) & 3)) << 4);
#pragma unroll
        for (int cc = 0; cc < NCT; ++cc) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const v4i B = *(const v4i*)(Vt + t * 8192 + cc * 1024);
#pragma unroll
                for (int s = 0; s < 5; ++s) {
                    if (s + t < 1) continue;
                    pacc[cc][s + t - 1] =
                        __builtin_amdgcn_mfma_i32_16x16x64_i8(Wd[s], B, pacc[cc][s + t - 1], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int cc = 0; cc < NCT; ++cc) EVs[cc] += TM->EV[16 * (NCT * hh + cc) + j];
        ++ep_tiles;
        tick(6);
        __syncthreads();  // every wave is done with the V buffer and the digit exchange
        if (it + 1 < ntiles) issue_v(it + 1);
    }

    // ---- certified final rounding, one (row, channel) at a time
    if (ntiles > 0) {
#pragma unroll 1
        for (int e = 0; e < 4 * NCT; ++e) {
            const int cc = e >> 2, i = e & 3;
            const double2 qd2 = *(const double2*)(scr + 2 * e);
            if (!(qd2.y >= 0.0)) continue;
            uint32_t bits = 0;
            if (!certify_round(qd2.x, qd2.y, P.out_fp32, &bits)) {
                failbits |= 1u << (8 * i + cc);
                continue;
            }
            const int lri = rbk * RPB + rg * 16 + 4 * g + i;
            if (lri < P.r_seg) {
                const int hq = hk * P.grp + lri % P.grp;
                const int64_t o = b * P.g.o_seq_stride + (int64_t)(lri / P.grp) * P.g.o_tok_stride +
                                  (int64_t)hq * P.g.o_head_stride + 16 * (NCT * hh + cc) + j;
                if (P.out_fp32) ((uint32_t*)P.out)[o] = bits;
                else ((uint16_t*)P.out)[o] = (uint16_t)bits;
            }
        }
    }
    if (TIMERS && lane == 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) atomicAdd((unsigned long long*)&P.timers[i], (unsigned long long)tclk[i]);
        atomicAdd((unsigned long long*)&P.timers[8], (unsigned long long)ntiles);
    }
    if (P.stats) {
        const int st5 = wave_sum_i(nunc_s), st6 = wave_sum_i(nunc_w), st8 = wave_sum_i(nslow);
        if (lane == 0) {
            if (st5) atomicAdd((unsigned long long*)&P.stats[5], (unsigned long long)st5);
            if (st6) atomicAdd((unsigned long long*)&P.stats[6], (unsigned long long)st6);
            if (st8) atomicAdd((unsigned long long*)&P.stats[8], (unsigned long long)st8);
        }
    }
    if (ntiles == 0) {
        // no key visible to any row of the block: every row is empty (+0) or a q domain error
        dom |= __shfl_xor(dom, 16, 64);
        dom |= __shfl_xor(dom, 32, 64);
        nv = 0;
        unc = 0;
    }
    // ---- row flags: a row fails when any channel of either wave of the pair failed
    {
        uint32_t fb = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint64_t bal = __ballot(((failbits >> (8 * i)) & 0xFF) != 0);
            if (((bal >> (16 * g)) & 0xFFFFull) != 0) fb |= 1u << i;
        }
        if (SPLIT == 2) {
            __syncthreads();  // s_x reuse
            s_x[w * 64 + lane].a = (int)fb;
            __syncthreads();
            fb |= (uint32_t)s_x[(w ^ 1) * 64 + lane].a;
        }
        failbits = fb;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int di = __shfl(dom, 4 * g + i, 64), ui = __shfl(unc, 4 * g + i, 64), nvr = __shfl(nv, 4 * g + i, 64);
        const bool fin = !di && !ui && ((failbits >> i) & 1);  // a final rounding failed
        const int flag = di ? 2 : ((ui || fin) ? 1 : 0);
        const int lri = rbk * RPB + rg * 16 + 4 * g + i;
        if (lri >= P.r_seg) continue;
        if (flag || nvr == 0) {
            const int hq = hk * P.grp + lri % P.grp;
            const int64_t o = b * P.g.o_seq_stride + (int64_t)(lri / P.grp) * P.g.o_tok_stride +
                              (int64_t)hq * P.g.o_head_stride + 16 * NCT * hh + j;
#pragma unroll
            for (int cc = 0; cc < NCT; ++cc) {
                if (P.out_fp32) ((uint32_t*)P.out)[o + 16 * cc] = 0u;
                else ((uint16_t*)P.out)[o + 16 * cc] = 0;
            }
        }
        if (j == 0 && hh == 0) {
            int ti;
            const int64_t gr = seg_row(P, b, hk, lri, &ti);
            P.flags[gr] = (uint8_t)flag;
            if (flag == 1) {
                const int slot = atomicAdd(P.wl_cnt, 1);
                P.wl[slot] = (int32_t)gr;
            }
            if (P.stats) {
                atomicAdd((unsigned long long*)&P.stats[0], 1ull);
                atomicAdd((unsigned long long*)&P.stats[10], 1ull);
                if (flag) atomicAdd((unsigned long long*)&P.stats[1], 1ull);
                if (flag == 2) atomicAdd((unsigned long long*)&P.stats[4], 1ull);
                if (fin) atomicAdd((unsigned long long*)&P.stats[7], 1ull);
            }
        }
    }
}

namespace {
// kernel shape: pair-split waves; 4 waves (32 rows, 1 wave per SIMD, 512 registers) by default,
// EA_PF_SHAPE=8 selects 8 waves (64 rows, 2 waves per SIMD)
int pf_rows_per_block() { return (getenv("EA_PF_SHAPE") && getenv("EA_PF_SHAPE")[0] == '8') ? 64 : 32; }
}  // namespace

int ea::ea_prefill_eligible(const ea_geometry& g, int grp, int* ntiles, int* nrb) {
    if (getenv("EA_PREFILL") && getenv("EA_PREFILL")[0] == '0') return 0;
    const bool force = getenv("EA_PREFILL") && getenv("EA_PREFILL")[0] == '1';
    if (g.head_dim != 128 || g.head_dim_v != 128) return 0;
    const int64_t r_seg = (int64_t)g.num_tokens * grp;
    if (!force && g.num_tokens < 64) return 0;
    if (r_seg >= (1 << 30) || (int64_t)g.max_seq_len + 64 >= (1 << 30)) return 0;
    const int rpb = pf_rows_per_block();
    *ntiles = (g.max_seq_len + 63) / 64;
    *nrb = (int)((r_seg + rpb - 1) / rpb);
    return 1;
}

int ea::ea_launch_prefill(const Params& P, hipStream_t st) {
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    std::call_once(once, [] {
        const void* fns[3] = {(const void*)ea_pf_main<2, 4, false>, (const void*)ea_pf_main<2, 4, true>,
                              (const void*)ea_pf_main<2, 8, false>};
        for (const void* f : fns)
            if (attr_err == hipSuccess)
                attr_err = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, PF_LDS);
    });
    if (attr_err != hipSuccess) return -100 - (int)attr_err;
    Params Pc = P;
    hipLaunchKernelGGL(ea_pf_qslice, dim3((unsigned)((P.rows + 63) / 64)), dim3(256), 0, st, Pc);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return -100 - (int)e;
    if (P.nseg > 0 && P.pf_ntiles > 0) {
        hipLaunchKernelGGL(ea_pf_kvslice, dim3((unsigned)(P.nseg * P.pf_ntiles)), dim3(256), 0, st, Pc);
        e = hipGetLastError();
        if (e != hipSuccess) return -100 - (int)e;
    }
    return 0;
}

int ea::ea_launch_prefill_main(const Params& P, hipStream_t st) {
    Params Pc = P;
    if (P.nseg > 0 && P.pf_nrb > 0) {
        const dim3 grid((unsigned)(P.nseg * P.pf_nrb));
        if (P.timers) hipLaunchKernelGGL((ea_pf_main<2, 4, true>), grid, dim3(256), PF_LDS, st, Pc);
        else if (pf_rows_per_block() == 64) hipLaunchKernelGGL((ea_pf_main<2, 8, false>), grid, dim3(512), PF_LDS, st, Pc);
        else hipLaunchKernelGGL((ea_pf_main<2, 4, false>), grid, dim3(256), PF_LDS, st, Pc);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return -100 - (int)e;
    }
    return 0;
}
