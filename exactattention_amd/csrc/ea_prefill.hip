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
#include "ea_pf_common.h"

using namespace ea;
using namespace ea::pf;

namespace {


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


// ------------------------------------------------------------------------------------------------
// Digits of NE consecutive bf16 elements held by one lane; the G = 128 / NE adjacent lanes of a
// group (lane & (G - 1)) cover a 128-element vector. Returns the vector's lsb (group-uniform) and
// the digit bytes (4 planes x NE bytes, as NE / 4 dwords per plane). K/V rows take NE = 32 (a quad
// per key); q rows NE = 8 (16 lanes per row: four times the lanes, a quarter of the chain).
// ------------------------------------------------------------------------------------------------
template <int NE>
struct SliceN {
    int lsb, bad, inex, need4, xmax;
    double amax, asum;
    uint32_t dig[4][NE / 4];
};
using Slice32 = SliceN<32>;

template <int G>
__device__ __forceinline__ int grp_max(int x) {
#pragma unroll
    for (int o = 1; o < G; o <<= 1) x = max(x, __shfl_xor(x, o, 64));
    return x;
}
template <int G>
__device__ __forceinline__ int grp_sum(int x) {
#pragma unroll
    for (int o = 1; o < G; o <<= 1) x += __shfl_xor(x, o, 64);
    return x;
}
template <int G>
__device__ __forceinline__ double grp_maxd(double x) {
#pragma unroll
    for (int o = 1; o < G; o <<= 1) x = fmax(x, __shfl_xor(x, o, 64));
    return x;
}
template <int G>
__device__ __forceinline__ double grp_sumd(double x) {
#pragma unroll
    for (int o = 1; o < G; o <<= 1) x += __shfl_xor(x, o, 64);
    return x;
}

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

// src: NE bf16 values (any alignment of 2 bytes); valid = false gives an all-zero vector.
// lost[c] (optional) receives 1 for each element that is not exact in 30 bits.
template <int NE>
__device__ __forceinline__ void slice_n(const uint16_t* src, bool valid, SliceN<NE>& S, int* lost = nullptr) {
    constexpr int G = 128 / NE;
    int m[NE], e[NE];
    int bad = 0, lead = INT_MIN;
    // the 2 NE bytes as 16-byte loads when they start on a 16-byte boundary (the usual cache
    // strides), else element by element
    uint32_t raw[NE / 2];
    if (valid && ((uintptr_t)src & 15) == 0) {
#pragma unroll
        for (int i = 0; i < NE / 8; ++i) {
            const uint4 v = ((const uint4*)src)[i];
            raw[4 * i] = v.x;
            raw[4 * i + 1] = v.y;
            raw[4 * i + 2] = v.z;
            raw[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NE / 2; ++i)
            raw[i] = valid ? ((uint32_t)src[2 * i] | ((uint32_t)src[2 * i + 1] << 16)) : 0u;
    }
#pragma unroll
    for (int k = 0; k < NE; ++k) {
        int bk;
        bf16_dec((raw[k >> 1] >> (16 * (k & 1))) & 0xFFFFu, &m[k], &e[k], &bk);
        bad |= bk;
        if (m[k] && !bk) lead = max(lead, lead_of(m[k], e[k]));
    }
    lead = grp_max<G>(lead);
    bad = grp_max<G>(bad);
    const int lsb = (lead == INT_MIN) ? 0 : lead - 29;
    int inex = 0, need4 = 0, xmax = 0;
    double amax = 0.0, asum = 0.0;
#pragma unroll
    for (int w4 = 0; w4 < NE / 4; ++w4) {
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
    S.inex = grp_sum<G>(inex);
    S.need4 = grp_max<G>(need4);
    S.xmax = grp_max<G>(xmax);
    S.amax = grp_maxd<G>(amax);
    S.asum = grp_sumd<G>(asum);  // integers below 2^41: exact in any order
}
__device__ __forceinline__ void slice32(const uint16_t* src, bool valid, Slice32& S, int* lost = nullptr) {
    slice_n<32>(src, valid, S, lost);
}

}  // namespace

// ------------------------------------------------------------------------------------------------
// q rows -> digit planes: 16 rows per block, 16 lanes per row (8 dims each: a short chain per lane,
// which is what a step of few rows, such as tree verification, waits on). Also clears the tier-2
// work-list counter (this is the step's first kernel on the prefill path).
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) ea_pf_qslice(Params P) {
    if (blockIdx.x == 0 && threadIdx.x <= EA_T2_BLOCKS) P.wl_cnt[threadIdx.x] = 0;
    const int q16 = threadIdx.x & 15;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    if (row >= P.rows) return;  // whole 16-lane groups leave together
    const int Hq = P.g.num_q_heads, T = P.g.num_tokens;
    const int64_t b = row / ((int64_t)T * Hq);
    const int t = (int)((row / Hq) % T), hq = (int)(row % Hq);
    const uint16_t* qr = P.q + b * P.g.q_seq_stride + (int64_t)t * P.g.q_tok_stride + (int64_t)hq * P.g.q_head_stride;
    SliceN<8> S;
    slice_n<8>(qr + 8 * q16, true, S);
    uint8_t* dst = P.pfq + row * 512 + 8 * q16;
#pragma unroll
    for (int sp = 0; sp < 4; ++sp) *(uint2*)(dst + 128 * sp) = make_uint2(S.dig[sp][0], S.dig[sp][1]);
    if (q16 == 0) {
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
    int seg, tile;
    if (P.kvd_begin) {
        // cache update: block i of a segment re-slices the i-th tile that holds an appended key
        seg = blockIdx.x / P.kvd_span;
        const int bs = seg / P.g.num_kv_heads;
        const int kb = max(P.kvd_begin[bs], 0), ke = P.kvd_end[bs];
        tile = kb / 64 + (int)(blockIdx.x % P.kvd_span);
        if (ke <= kb || tile * 64 >= ke || tile >= P.pf_ntiles) return;  // uniform: the whole block
    } else {
        seg = blockIdx.x / P.pf_ntiles;
        tile = blockIdx.x % P.pf_ntiles;
    }
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
            TM->kA[key] = ldexp(S.amax, S.lsb);  // in absolute units: the score bound needs no rescale
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
        TM->pad = 0;
        TM->EVt = 0.5 * (0x1p38 + 1.0) * (double)tot;
    }
}

// ------------------------------------------------------------------------------------------------
// Main kernel. Block = NWB waves over 32 consecutive rows (tokens x query heads of one KV head):
// two row groups rg of 16 rows, SPLIT = NWB / 2 waves each. Wave hh of a row group takes the
// scores and weights of key groups kt = NKT hh .. NKT hh + NKT - 1 of each 64-key tile and the
// P.V sums of channel tiles ct = NCT hh .. NCT hh + NCT - 1 (NWB = 8: one key group and two
// channel tiles per wave; NWB = 4: two and four). Lane (g = lane / 16, j = lane % 16):
//   score layout  row j, keys 16 kt + 4 g + i (i = 0..3)
//   P.V layout    rows 4 g + i, channels 16 ct + j
// Software pipeline, one step per tile it, two barriers:
//   B1    K(it), its metadata and V(it-1) landed; the row maxima of tile it-1 are in sX
//         score MFMAs of tile it (K planes and q digits from LDS); while they run, the base move
//         (epoch fold when a base moves) and the weight digits of tile it-1 to sWD
//   B2    every wave has read the K planes of tile it and written its digits: row group 0's
//         waves issue the DMAs of K(it+1) with its metadata and of V(it) while row group 1's go
//         on; fp64 scores; P.V MFMAs of tile it-1 (digits from sWD), certification of tile it,
//         cold path; row maxima of tile it to sX
// V and the metadata are double-buffered (the two parities are two copies of the step). The DMAs
// are issued as inline asm, so the compiler adds no waits of its own; barriers are s_barrier after
// lgkmcnt(0) (no vmcnt(0): DMAs stay in flight across them) and the DMA waits are vmcnt(NKI)
// before B1 (K(it) and its metadata) and vmcnt(0) before B2 (V(it-1)).
// ------------------------------------------------------------------------------------------------
struct PfX {
    int32_t a, b;
    double c;
};

// LDS layout (dynamic): the DMA targets first, all below 104 KB
constexpr int PF_OFF_K = 0;
constexpr int PF_OFF_V0 = 32768;
constexpr int PF_OFF_V1 = 65536;
constexpr int PF_OFF_M0 = 98304;
constexpr int PF_OFF_M1 = PF_OFF_M0 + 4096;
constexpr int PF_QROW = 528;                 // q digit row stride in LDS: 512 bytes + 16 of padding
constexpr int PF_OFF_Q = PF_OFF_M1 + 4096;  // 32 rows x PF_QROW bytes
constexpr int PF_OFF_T = PF_OFF_Q + 32 * PF_QROW;
constexpr int PF_OFF_WD = PF_OFF_T + 4096;  // 5 planes x 4 key groups x 2 row groups x 64 lanes x 4 B
constexpr int PF_OFF_X = PF_OFF_WD + 10240;  // up to 8 waves x 64 lanes x 16 bytes
constexpr int PF_OFF_KEND = PF_OFF_X + 8192;
constexpr int PF_LDS = PF_OFF_KEND + 16;

template <int N>
struct PfPar {
    static constexpr int value = N;
};

template <int NWB, bool TIMERS>
__global__ void __launch_bounds__(64 * NWB, 1) ea_pf_main(Params P) {
    // phase clocks (TIMERS build): shader cycles summed over waves into P.timers[i]. Per tile:
    // [14] DMA wait before B1, [0] B1, [1] EV reads and score MFMAs, [2] base move and weight
    // digits, [3] B2, DMA issue, fp64 scores and digit reads, [4] pair metadata, P.V and
    // certification, [5] cold path, [6] pair exchange, [7] the rest. Per block: [15] prologue,
    // [9] drain, [10] row totals, [11] earlier epochs and reciprocals, [12] normal-range rounding
    // of every entry, [13] the general test for the rest. [8] counts tiles (lane 0 of each wave).
    uint64_t tclk[16] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    uint64_t tprev = TIMERS ? __builtin_amdgcn_s_memtime() : 0;
    auto tick = [&](int ph) __attribute__((always_inline)) {
        if (TIMERS) {
            const uint64_t t = __builtin_amdgcn_s_memtime();
            tclk[ph] += t - tprev;
            tprev = t;
        }
    };
    // the clocks into P.timers, once per wave (slot 8 counts the wave's tiles)
    auto flush_timers = [&](int ntile) __attribute__((always_inline)) {
        if (TIMERS && (threadIdx.x & 63) == 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (i != 8) atomicAdd((unsigned long long*)&P.timers[i], (unsigned long long)tclk[i]);
            atomicAdd((unsigned long long*)&P.timers[8], (unsigned long long)ntile);
        }
    };
    constexpr int SPLIT = NWB / 2;         // waves per row group of 16 rows
    constexpr int RPB = 16 * NWB / SPLIT;  // rows per block (32)
    constexpr int NKT = 4 / SPLIT;         // key groups of 16 per wave
    constexpr int NCT = 8 / SPLIT;         // channel tiles of 16 per wave
    constexpr int NKI = 64 / NWB;          // K (and V) DMA instructions per issuing wave and tile
    extern __shared__ __align__(16) unsigned char smem[];
    uint8_t* const sK = smem + PF_OFF_K;     // K planes of the current tile
    uint8_t* const sV0 = smem + PF_OFF_V0;   // V planes, even tiles
    uint8_t* const sV1 = smem + PF_OFF_V1;   // V planes, odd tiles
    uint8_t* const sM0 = smem + PF_OFF_M0;   // tile metadata, even tiles
    uint8_t* const sM1 = smem + PF_OFF_M1;   // tile metadata, odd tiles
    uint8_t* const sQ = smem + PF_OFF_Q;     // q digits of the block's rows
    double* const sT1 = (double*)(smem + PF_OFF_T);  // T1 * 2^23, then T2
    double* const sT2 = sT1 + 256;
    uint32_t* const sWD = (uint32_t*)(smem + PF_OFF_WD);  // weight digits [wave][plane 5][2][lane]
    PfX* const sX = (PfX*)(smem + PF_OFF_X);              // pair exchange [wave][lane]
    int& s_kend = *(int*)(smem + PF_OFF_KEND);
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = w / SPLIT, hh = w % SPLIT;
    const int g = lane >> 4, j = lane & 15;
    const int nseg = P.nseg;
    const int seg = blockIdx.x % nseg;
    const int split = (int)(blockIdx.x / nseg) % P.pf_nsplit;  // key split (tile range) of the block
    const int rbk = P.pf_nrb - 1 - (int)(blockIdx.x / nseg) / P.pf_nsplit;
    const int Hkv = P.g.num_kv_heads;
    const int64_t b = seg / Hkv;
    const int hk = seg % Hkv;
    // the segment's K/V tiles: its own in the workspace, or its slot's in the caller's cache
    const int64_t kseg = (P.pf_kv_cached && P.pf_kv_slot) ? (int64_t)P.pf_kv_slot[b] * Hkv + hk : (int64_t)seg;
    const int T = P.g.num_tokens;
    constexpr int WDS = 5 * NKT * 64;  // digit dwords per wave: [plane 5][NKT][lane 64]
    uint32_t* const wd_w = sWD + w * WDS + lane;                    // this wave's digit planes
    const uint32_t* const wd_r = sWD + (rg * SPLIT) * WDS + lane;  // the row group's, by key group
    // per-lane scratch: fp64 sums of completed epochs, then the final quotients
    double* const scr = P.pfscr + (((int64_t)blockIdx.x * NWB + w) * 64 + lane) * (8 * NCT);

    if (tid == 0) s_kend = 0;
    if (tid < 256) {
        sT1[tid] = u64_as_f64(EA_T1_BITS[tid]) * 8388608.0;  // 2^23: exact
        sT2[tid] = u64_as_f64(EA_T2_BITS[tid]);
    }
    // step 0 runs the P.V of "tile -1" on zero weight digits and adds the zero EV of sM1
    for (int c = tid; c < NWB * WDS; c += 64 * NWB) sWD[c] = 0u;
    if (tid < 128) ((PfTileMeta*)sM1)->EV[tid] = 0.0;
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
    // keys below kvmin are visible to every row of the wave (and of its partner)
    const int kvmin = wave_min_i(rvalid ? min(kvl, slen) : INT_MAX);
    __syncthreads();  // s_kend initialised
    {
        const int kw = wave_max_i(ve);
        if (lane == 0) atomicMax(&s_kend, kw);
    }
    // q digits of the block's rows into LDS: [row][plane 4][128 bytes] with rows PF_QROW = 528
    // bytes apart, so the 16 rows a 16-lane group reads start 4 banks apart (132 dwords = 4 mod 64)
    // and a 16-byte read per lane touches every bank once; rows past the segment repeat its last row
    for (int c = tid; c < RPB * 32; c += 64 * NWB) {
        const int r = c >> 5, q16 = c & 31;
        const int lrr = min(rbk * RPB + r, P.r_seg - 1);
        int tt;
        const int64_t gr = seg_row(P, b, hk, lrr, &tt);
        *(uint4*)(sQ + r * PF_QROW + q16 * 16) = *(const uint4*)(P.pfq + gr * 512 + q16 * 16);
    }
    // this lane's q digits (B operand of the score MFMA): row j, dims 64 h + 16 g .. + 15, plane s:
    // chunk 8 s + 4 h + g of the row
    const uint8_t* const qlds = sQ + (rg * 16 + j) * PF_QROW;
    const uint8_t* const qb[2] = {qlds + (g << 4), qlds + ((4 + g) << 4)};
    // K operand: key 16 kt + j, chunk (4 h + g) ^ (j & 7), plane t at + 8192 t, key group at + 2048 kt
    const uint8_t* const kb[2] = {sK + j * 128 + ((g ^ (j & 7)) << 4), sK + j * 128 + (((4 + g) ^ (j & 7)) << 4)};
    const PfQMeta qm = ((const PfQMeta*)P.pfqm)[grow];
    const bool needq = __ballot(rvalid && (qm.flags & 1)) != 0;
    // the score bound per pair is adq * kA 2^lk: |a| times the fold error factor 6.01 u times
    // sum_i A_q,i, with 2^-48 of slack for the roundings of this product and of adq * kAs
    const double adq = fabs(qm.a) * (6.01 * 0x1p-53) * qm.qA * (1.0 + 0x1p-48);
    const double aqL = fabs(qm.a) * 0.5 * (double)((qm.flags >> 8) & 0xFF);
    const double aqX = fabs(qm.a) * 0.5 * (qm.qX + 1.0);
    const bool lossy_q = __ballot(rvalid && ((qm.flags >> 8) & 0xFF)) != 0;
    const bool qbad = (qm.flags & 2) != 0;
    int dom = (rvalid && qbad) ? 1 : 0;  // NaN/inf in q: a domain error (docs/SPEC.md)
    int unc = 0;
    int nslow = 0, nunc_s = 0, nunc_w = 0;
    // wave-uniform event counts, added to the stats once at the end: an atomic inside the tile loop
    // would make the next wait for vector memory (vmcnt) also wait for its round trip
    int nfold = 0, ncold = 0;
    __syncthreads();  // s_kend final, tables and q digits visible
    const int kend = s_kend;
    const int ntiles = (kend + 63) >> 6;
    // this block's key split: tiles [t0, t1) of the rows' visible range
    const int t0 = min(split * P.pf_tps, ntiles), t1 = min(t0 + P.pf_tps, ntiles);
    const int nt = t1 - t0;
    const double* const T1s = sT1;
    const double* const T2 = sT2;

    // tile DMA: only the SPLIT waves of row group 0 issue, each NKI instructions of 1 KB for the K
    // (or V) planes and its share of the 4 KB of metadata. A wave stalls at a DMA instruction until
    // the texture path accepts it (about 2,000 cycles for a tile's 68 instructions); with one
    // issuing wave per SIMD the other wave on that SIMD, of row group 1, runs its P.V and
    // certification meanwhile instead of stalling beside it. Issued through pf_dma (inline asm),
    // so the compiler inserts no waits of its own before the LDS reads: every read of a DMA'd
    // buffer follows an explicit vmcnt wait for that buffer (row group 1 has nothing in flight).
    auto rsrc = [&](int tile) __attribute__((always_inline)) {
        const uint64_t src = (uint64_t)(P.pfkv + (kseg * P.pf_ntiles + tile) * EA_PF_TILE_BYTES);
        v4i r = {(int)(uint32_t)src, (int)((uint32_t)(src >> 32) & 0xFFFFu), EA_PF_TILE_BYTES, 0x00020000};
        r.x = __builtin_amdgcn_readfirstlane(r.x);
        r.y = __builtin_amdgcn_readfirstlane(r.y);
        return r;
    };
    const int vlane = lane * 16;  // one lane offset; the per-instruction offset goes in soffset
    const uint32_t aK = lds_addr(sK), aV0 = lds_addr(sV0), aV1 = lds_addr(sV1), aM0 = lds_addr(sM0),
                   aM1 = lds_addr(sM1);
    auto issue_k = [&](int tile, uint32_t mdst) __attribute__((always_inline)) {
        if (rg != 0) return;
        const v4i rs = rsrc(tile);
#pragma unroll
        for (int q = 0; q < NKI; ++q) {
            const int off = (q * SPLIT + hh) * 1024;
            pf_dma(rs, aK + off, vlane, off);
        }
#pragma unroll
        for (int m = hh; m < 4; m += SPLIT) pf_dma(rs, mdst + m * 1024, vlane, EA_PF_META_OFF + m * 1024);
    };
    auto issue_v = [&](int tile, uint32_t vdst) __attribute__((always_inline)) {
        if (rg != 0) return;
        const v4i rs = rsrc(tile);
#pragma unroll
        for (int q = 0; q < NKI; ++q) {
            const int off = (q * SPLIT + hh) * 1024;
            pf_dma(rs, vdst + off, vlane, 32768 + off);
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

    // fp64 value of the int32 P.V accumulators of (channel tile cc, row 4 g + i) in units 2^base,
    // and the bound of everything the epoch left out: fold roundings (6.02 u sum |acc|), inexact V
    // elements (EVs), the omitted digit pair (0, 0) (2^20 per tile), weight roundings below the
    // base (fr_i = 2^29 per key: 2^30 / 2)
    auto epoch_sum = [&](int cc, int i, double fr_i, double omit, double* en) __attribute__((always_inline)) {
        double h = (double)pacc[cc][6][i], ha = fabs(h);
#pragma unroll
        for (int k = 5; k >= 0; --k) {
            const double a = (double)pacc[cc][k][i];
            h = __fma_rn(h, 256.0, a);
            ha = __fma_rn(ha, 256.0, fabs(a));
        }
        *en = 6.02 * 0x1p-53 * (ha * 256.0) + EVs[cc] + omit + fr_i;
        return h * 256.0;
    };
    // ---- fold the epoch into the per-lane fp64 sums in scr, rescaled to the new bases nb
    auto fold = [&](int nf_pair, int nb) __attribute__((always_inline)) {
        ++nfold;
        int nf = nf_pair + __shfl_xor(nf_pair, 16, 64);
        nf += __shfl_xor(nf, 32, 64);
        double fr[4];
        int bo[4], bn[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            bo[i] = __shfl(base, 4 * g + i, 64);
            bn[i] = __shfl(nb, 4 * g + i, 64);
            fr[i] = 0x1p29 * (double)__shfl(nf, 4 * g + i, 64);
        }
        nfrac = 0;
        const double omit = (double)ep_tiles * 0x1p20;  // pair (0, 0): 64 keys x 2^14
#pragma unroll
        for (int cc = 0; cc < NCT; ++cc) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                double en;
                double nn = epoch_sum(cc, i, fr[i], omit, &en);
                double2* sp = (double2*)(scr + 2 * (4 * cc + i));
                if (had_fold) {
                    const double2 o = *sp;
                    nn += o.x;
                    en += o.y;
                }
                en += fabs(nn) * 0x1p-52;
                if (bo[i] != INT_MIN && bn[i] != bo[i]) {
                    const int dsh = max(bo[i] - bn[i], -1100);
                    nn = ldexp(nn, dsh);
                    en = ldexp(en, dsh) + 0x1p-1074;
                }
                *sp = make_double2(nn, en);
#pragma unroll
                for (int k = 0; k < 7; ++k) pacc[cc][k][i] = 0;
            }
        }
#pragma unroll
        for (int cc = 0; cc < NCT; ++cc) EVs[cc] = 0.0;
        ep_tiles = 0;
        had_fold = true;
        wait_vm<0>();  // the scr stores are complete (keeps the DMA counts exact)
    };

    // ---- P.V of the tile whose digits are in sWD and V planes in vbuf: pacc[cc][s + t - 1] +=
    // W digits s x V digits t (all pairs but (0, 0)). Channel 16 (NCT hh + cc) + j: the 16-byte
    // slot swizzle (ch >> 1) & 3 = (j >> 1) & 3 does not depend on cc, so every read is one lane
    // base plus a constant.
    auto pv_mfma = [&](const v4i (&Wd)[5], const uint8_t* vbuf, int c0, int c1) __attribute__((always_inline)) {
        const uint8_t* Vt = vbuf + (16 * NCT * hh + j) * 64 + ((g ^ ((j >> 1) & 3)) << 4);
#pragma unroll
        for (int cc = c0; cc < c1; ++cc) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const v4i B = *(const v4i*)(Vt + t * 8192 + cc * 1024);
#pragma unroll
                for (int s = 0; s < 5; ++s) {
                    if (s + t < 1) continue;
                    pacc[cc][s + t - 1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(Wd[s], B, pacc[cc][s + t - 1], 0, 0, 0);
                }
            }
        }
    };
    auto read_wd = [&](v4i (&Wd)[5]) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < 5; ++s)
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) Wd[s][kt] = (int)wd_r[(kt / NKT) * WDS + (s * NKT + kt % NKT) * 64];
    };

    // ---- weights of the previous tile (certified in the previous step) and this wave's row maxima
    v4i cMk[NKT], cEk[NKT], cvl[NKT];
    int cgm = INT_MIN;
    // ---- after B1: the row group's maxima of the previous tile are in sX. Move the base (folding
    // the epoch first when it moves or is 256 tiles old), add the previous tile's inexact-V
    // counts, then write the previous tile's weight digits (A operand of the P.V MFMA) to sWD.
    auto rebase_digits = [&](const double (&evp)[NCT]) __attribute__((always_inline)) {
        int gm = cgm;
        int nf_pair = nfrac;  // the row group's keys (all SPLIT waves) of the epoch
#pragma unroll
        for (int o = 1; o < SPLIT; ++o) {
            const PfX x = sX[(rg * SPLIT + (hh + o) % SPLIT) * 64 + lane];
            gm = max(gm, x.a);
            nf_pair += x.b;
        }
        // the base moves when a weight would exceed 2^38 (G - base > 14 for G = E + vlsb)
        const bool need_rb = gm != INT_MIN && (base == INT_MIN || gm > base + 14);
        const int nb = need_rb ? gm - 10 : base;
        if (ep_tiles > 0 && (__ballot(need_rb) != 0 || ep_tiles >= 256)) fold(nf_pair, nb);
#pragma unroll
        for (int cc = 0; cc < NCT; ++cc) EVs[cc] += evp[cc];
        if (nb != base && base != INT_MIN) z = ldexp(z, max(base - nb, -1100));
        base = nb;
    #pragma unroll
            for (int kk = 0; kk < NKT; ++kk) {
                uint32_t L[4], H[4];
    #pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int Mp = cMk[kk][i];
                    const int sc = cEk[kk][i] - base;
                    const double md = (double)Mp;
                    const double wsc = ldexp(md, sc + cvl[kk][i]);  // <= 2^38
                    z += ldexp(md, sc);                             // md = 0 for masked pairs
                    nv += Mp ? 1 : 0;
                    nfrac += (Mp && sc + cvl[kk][i] < 0) ? 1 : 0;
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
                uint32_t* wd = wd_w + kk * 64;
                wd[0 * 64 * NKT] = __builtin_amdgcn_perm(a23, a01, 0x05040100u) ^ 0x80808080u;
                wd[1 * 64 * NKT] = __builtin_amdgcn_perm(a23, a01, 0x07060302u) ^ 0x80808080u;
                wd[2 * 64 * NKT] = __builtin_amdgcn_perm(b23, b01, 0x05040100u) ^ 0x80808080u;
                wd[3 * 64 * NKT] = __builtin_amdgcn_perm(b23, b01, 0x07060302u) ^ 0x80808080u;
                wd[4 * 64 * NKT] = __builtin_amdgcn_perm(e23, e01, 0x05040100u) ^ 0x80808080u;
            }
    };

    // ---- one pipeline step, tile it (B1, score MFMAs beside the base move and digits of tile
    // it-1, B2, DMAs of K(it+1) and V(it), P.V of tile it-1, certification of tile it)
    auto step = [&](auto par, int it) __attribute__((always_inline)) {
        constexpr int PA = decltype(par)::value;
        const uint8_t* const sVp = PA ? sV0 : sV1;  // V(it - 1)
        const uint32_t aVc = PA ? aV1 : aV0;        // V(it) loads into the buffer V(it - 2) used
        const PfTileMeta* const TMc = (const PfTileMeta*)(PA ? sM1 : sM0);
        const PfTileMeta* const TMp = (const PfTileMeta*)(PA ? sM0 : sM1);
        const uint32_t aMn = PA ? aM0 : aM1;        // metadata of tile it + 1
        const bool k_next = it + 1 < t1;
        tick(7);
        // K(it) and its metadata landed. V(it - 1), issued after them, is first read after B2 and
        // is waited for there; at the first tile nothing else is in flight.
        if (it > t0) wait_vm<NKI>();
        else wait_vm<0>();
        tick(14);
        pf_bar();      // B1
        tick(0);
        const int tfl = TMc->tfl;
        // the previous tile's inexact-V counts, read before its metadata buffer is reloaded
        double evp[NCT];
#pragma unroll
        for (int cc = 0; cc < NCT; ++cc) evp[cc] = TMp->EV[16 * (NCT * hh + cc) + j];
        // ---- score MFMAs of tile it, then (while they run) the previous tile's base move and
        // weight digits
        v4i sacc[NKT][7];
#pragma unroll
        for (int kk = 0; kk < NKT; ++kk)
#pragma unroll
            for (int k = 0; k < 7; ++k) sacc[kk][k] = (v4i){0, 0, 0, 0};
        const bool wide = needq || ((tfl >> (NKT * hh)) & ((1 << NKT) - 1));
        auto scores = [&]() __attribute__((always_inline)) {
            if (wide) {
#pragma unroll
                for (int kk = 0; kk < NKT; ++kk) score_mfma<true>(kb, qb, NKT * hh + kk, sacc[kk]);
            } else {
#pragma unroll
                for (int kk = 0; kk < NKT; ++kk) score_mfma<false>(kb, qb, NKT * hh + kk, sacc[kk]);
            }
        };
        scores();
        tick(1);
        if (it > t0) rebase_digits(evp);
        tick(2);
        // every wave has read the K planes of tile it and written the weight digits of tile it - 1,
        // and V(it - 1) has landed: K(it + 1) with its metadata and V(it) start loading
        wait_vm<0>();
        pf_bar();
        if (k_next) issue_k(it + 1, aMn);
        issue_v(it, aVc);
        v4i lk4[NKT];
        double xs[NKT][4];
#pragma unroll
        for (int kk = 0; kk < NKT; ++kk) {
            lk4[kk] = *(const v4i*)&TMc->lsbk[16 * (NKT * hh + kk) + 4 * g];
            score_fold(sacc[kk], lk4[kk], xs[kk]);
        }
        v4i Wd[5];
        read_wd(Wd);  // zero at it = t0
        if (it > t0) ++ep_tiles;
        tick(3);
        // ---- per-pair metadata, score bounds and visibility of tile it
        v4i vl4[NKT];
        double adel[NKT][4];
#pragma unroll
        for (int kk = 0; kk < NKT; ++kk) {
            const int kt = NKT * hh + kk;
            vl4[kk] = *(const v4i*)&TMc->vlsb[16 * kt + 4 * g];
            const double2 kA01 = *(const double2*)&TMc->kA[16 * kt + 4 * g];
            const double2 kA23 = *(const double2*)&TMc->kA[16 * kt + 4 * g + 2];
            adel[kk][0] = adq * kA01.x;
            adel[kk][1] = adq * kA01.y;
            adel[kk][2] = adq * kA23.x;
            adel[kk][3] = adq * kA23.y;
        }
        if (lossy_q || (tfl & 32)) {
            // elements rounded at slicing: |q_i - Q_i| <= 2^lsbq / 2 and the same for k
#pragma unroll
            for (int kk = 0; kk < NKT; ++kk)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = 16 * (NKT * hh + kk) + 4 * g + i;
                    const double e = __fma_rn(aqL, TMc->kX[key] + 1.0, (double)(TMc->kfl[key] >> 8) * aqX);
                    adel[kk][i] = (adel[kk][i] + ldexp(e, lk4[kk][i])) * (1.0 + 0x1p-50);
                }
        }
        uint32_t vism = rvalid ? 0xFFu : 0u;  // bit 4 kk + i: pair visible
        if (!((it + 1) * 64 <= kvmin)) {
            vism = 0;
#pragma unroll
            for (int kk = 0; kk < NKT; ++kk)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int n = it * 64 + 16 * (NKT * hh + kk) + 4 * g + i;
                    const int ti = n - tbase;
                    const bool intree = ((unsigned)ti < 64u) & (((tmk >> (ti & 63)) & 1ull) != 0);
                    vism |= ((n < slen) & ((n < kvl) | intree)) ? (1u << (4 * kk + i)) : 0u;
                }
        }
        if (tfl & 16) {
            // NaN/inf in a key's K or V row: a domain error for the rows that see it
#pragma unroll
            for (int kk = 0; kk < NKT; ++kk)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int bit = 1 << (4 * kk + i);
                    if (TMc->kfl[16 * (NKT * hh + kk) + 4 * g + i] & 1) {
                        if (vism & bit) dom = 1;
                        vism &= ~(uint32_t)bit;
                    }
                }
        }
        // ---- P.V of tile it - 1 (zero digits at it = t0) beside the certification of tile it
        v4i Mk[NKT], Ek[NKT];
        uint32_t slowmask = 0;  // pairs the fast path left undecided (cold path below)
        int gm = INT_MIN;
#pragma unroll
        for (int kk = 0; kk < NKT; ++kk) {
            pv_mfma(Wd, sVp, kk * (NCT / NKT), (kk + 1) * (NCT / NKT));
            int M[4], E[4];
            bool ok[4];
            cert4(xs[kk], adel[kk], qm.a, T1s, T2, M, E, ok);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool vis = (vism >> (4 * kk + i)) & 1;
                const bool good = vis & ok[i];
                slowmask |= (vis & !ok[i]) ? (1u << (4 * kk + i)) : 0u;
                Mk[kk][i] = good ? M[i] : 0;
                Ek[kk][i] = E[i];
                gm = max(gm, good ? E[i] + vl4[kk][i] : INT_MIN);
            }
        }
        tick(4);
        // ---- cold path: exact decision for the pairs the fast path left undecided. The exact
        // integer score comes from the tile's digit planes (no bf16 reads); only pairs whose
        // digits are inexact (elements rounded at slicing) read the bf16 inputs.
        if (__builtin_expect(__ballot(slowmask != 0) != 0, 0)) {
            ++ncold;
            const int8_t* Kg = (const int8_t*)(P.pfkv + (kseg * P.pf_ntiles + it) * EA_PF_TILE_BYTES);
            for (int p = 0; p < 4 * NKT; ++p) {
                if (!((slowmask >> p) & 1)) continue;
                const int kk = p >> 2, i = p & 3;
                const int key = 16 * (NKT * hh + kk) + 4 * g + i;
                const int n = it * 64 + key;
                const int kf = TMc->kfl[key];
                ++nslow;
                // the pair's exact decision, out of line: from the tile's digit planes when every
                // element was sliced exactly, else from the bf16 inputs
                const int mode = qbad ? 2 : ((!((qm.flags >> 8) & 0xFF) && !(kf >> 8)) ? 0 : 1);
                const uint16_t* qr = nullptr;
                const uint16_t* kr = nullptr;
                if (mode == 1) {
                    qr = P.q + b * P.g.q_seq_stride + (int64_t)tq * P.g.q_tok_stride +
                         (int64_t)(hk * P.grp + lrc % P.grp) * P.g.q_head_stride;
                    kr = P.k + kv_off(P, b, n, hk, 0);
                }
                const int3 cw = pf_cold_pair(mode, qlds, 0, (const uint8_t*)Kg + key * 128, key & 7, qr, kr, P.am,
                                             P.ae + qm.lsb + TMc->lsbk[key], P.alpha, T1s, T2);
                const bool live = cw.x == 0;
                const int32_t M = cw.y, E = cw.z;
                if (cw.x == 2) dom = 1;
                if (cw.x == 3) {
                    unc = 1;
                    ++nunc_s;
                }
                if (cw.x == 4) {
                    unc = 1;
                    ++nunc_w;
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
                if (live) gm = max(gm, E + TMc->vlsb[key]);
            }
        }
        tick(5);
        // ---- the row's largest weight in this tile (this wave's 4 lanes of the row), for the
        // row group's exchange after the next B1
        gm = max(gm, __shfl_xor(gm, 16, 64));
        gm = max(gm, __shfl_xor(gm, 32, 64));
        sX[w * 64 + lane] = PfX{gm, nfrac, 0.0};
        cgm = gm;
#pragma unroll
        for (int kk = 0; kk < NKT; ++kk) {
            cMk[kk] = Mk[kk];
            cEk[kk] = Ek[kk];
            cvl[kk] = vl4[kk];
        }
        tick(6);
    };

    wait_vm<0>();  // the prologue's global loads: from here on vmcnt counts DMAs (and folds)
    if (nt > 0) issue_k(t0, aM0);
    tick(15);
    for (int it = t0; it < t1; it += 2) {
        step(PfPar<0>{}, it);
        if (it + 1 < t1) step(PfPar<1>{}, it + 1);
    }
    tick(7);
    // ---- drain: digits and P.V of the last tile
    if (nt > 0) {
        wait_vm<0>();
        pf_bar();
        const bool odd = (nt - 1) & 1;
        const PfTileMeta* TMl = (const PfTileMeta*)(odd ? sM1 : sM0);
        double evp[NCT];
#pragma unroll
        for (int cc = 0; cc < NCT; ++cc) evp[cc] = TMl->EV[16 * (NCT * hh + cc) + j];
        rebase_digits(evp);
        pf_bar();
        v4i Wd[5];
        read_wd(Wd);
        ++ep_tiles;
        pv_mfma(Wd, odd ? sV1 : sV0, 0, NCT);
    }
    tick(9);
    // ---- row totals for the final rounding: this wave's 4 lanes of the row, then the partner
    z += __shfl_xor(z, 16, 64);
    z += __shfl_xor(z, 32, 64);
    nv += __shfl_xor(nv, 16, 64);
    nv += __shfl_xor(nv, 32, 64);
    dom |= __shfl_xor(dom, 16, 64);
    dom |= __shfl_xor(dom, 32, 64);
    unc |= __shfl_xor(unc, 16, 64);
    unc |= __shfl_xor(unc, 32, 64);
    sX[w * 64 + lane] = PfX{nv, nfrac | (dom << 24) | (unc << 25), z};
    pf_bar();
    int nf_pair = nfrac;
    {
#pragma unroll
        for (int o = 1; o < SPLIT; ++o) {
            const PfX x = sX[(rg * SPLIT + (hh + o) % SPLIT) * 64 + lane];
            nv += x.a;
            nf_pair += x.b & 0xFFFFFF;
            dom |= (x.b >> 24) & 1;
            unc |= (x.b >> 25) & 1;
            z += x.c;
        }
    }
    tick(10);
    if (P.pf_nsplit > 1) {
        // ---- key splits: this split's (N, bound) per (row, channel) and (base, nv, flags, Z) per
        // row, in units 2^base; ea_pf_combine merges the splits and rounds. Every record a
        // combine reads is written here (a split with no tile writes nv = 0 and its flags).
        PfPart* const parts = (PfPart*)P.pf_part;
        double2* const ent = (double2*)(parts + (int64_t)P.pf_nsplit * P.rows);
        if (nt > 0) {
            int nf = nf_pair + __shfl_xor(nf_pair, 16, 64);
            nf += __shfl_xor(nf, 32, 64);
            const double omit = (double)ep_tiles * 0x1p20;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int lri = rbk * RPB + rg * 16 + 4 * g + i;
                if (lri >= P.r_seg) continue;
                int ti;
                const int64_t gr = seg_row(P, b, hk, lri, &ti);
                const double fri = 0x1p29 * (double)__shfl(nf, 4 * g + i, 64);
#pragma unroll
                for (int cc = 0; cc < NCT; ++cc) {
                    double en;
                    double nn = epoch_sum(cc, i, fri, omit, &en);
                    if (had_fold) {
                        const double2 o = *(const double2*)(scr + 2 * (4 * cc + i));
                        nn += o.x;
                        en += o.y;
                    }
                    en += fabs(nn) * 0x1p-52;
                    ent[((int64_t)split * P.rows + gr) * 128 + 16 * (NCT * hh + cc) + j] = make_double2(nn, en);
                }
            }
        }
        if (g == 0 && hh == 0 && rvalid) {
            PfPart pr;
            pr.base = nv > 0 ? base : INT_MIN;
            pr.nv = nv;
            pr.fl = (dom ? 1 : 0) | (unc ? 2 : 0);
            pr.pad = 0;
            pr.z = z;
            pr.pad2 = 0.0;
            parts[(int64_t)split * P.rows + grow] = pr;
        }
        if (P.stats) {
            const int st5 = wave_sum_i(nunc_s), st6 = wave_sum_i(nunc_w), st8 = wave_sum_i(nslow);
            // rows are counted once, by the blocks of split 0
            const int cr = wave_sum_i((split == 0 && g == 0 && hh == 0 && rvalid) ? 1 : 0);
            if (lane == 0) {
                if (st5) atomicAdd((unsigned long long*)&P.stats[5], (unsigned long long)st5);
                if (st6) atomicAdd((unsigned long long*)&P.stats[6], (unsigned long long)st6);
                if (st8) atomicAdd((unsigned long long*)&P.stats[8], (unsigned long long)st8);
                if (nfold) atomicAdd((unsigned long long*)&P.stats[11], (unsigned long long)nfold);
                if (ncold) atomicAdd((unsigned long long*)&P.stats[12], (unsigned long long)ncold);
                if (cr) {
                    atomicAdd((unsigned long long*)&P.stats[0], (unsigned long long)cr);
                    atomicAdd((unsigned long long*)&P.stats[10], (unsigned long long)cr);
                }
            }
        }
        flush_timers(nt);  // loop phases, prologue, drain and row totals (no final rounding here)
        return;
    }
    // ---- the last epoch plus the earlier ones, then RN(N/Z) per (row, channel), certified:
    // q = N * RN(1/Z) (two roundings: below 2^-51.9 |q|, inside the 2^-51 |q| term) and
    // delta >= |N/Z - q| from the N bound en and the Z bound eZ
    if (nt > 0) {
        double2 prev[4 * NCT];
#pragma unroll
        for (int e = 0; e < 4 * NCT; ++e) prev[e] = had_fold ? *(const double2*)(scr + 2 * e) : make_double2(0.0, 0.0);
        int nf = nf_pair + __shfl_xor(nf_pair, 16, 64);
        nf += __shfl_xor(nf, 32, 64);
        double fr[4], Zr[4], eZr[4], rz[4], rze[4];
        bool skip[4], live[4];  // skip: empty row, domain error or undecided pair (no output here)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            fr[i] = 0x1p29 * (double)__shfl(nf, 4 * g + i, 64);
            Zr[i] = __shfl(z, 4 * g + i, 64);
            const int nvr = __shfl(nv, 4 * g + i, 64);
            eZr[i] = (double)(nvr + 8) * PF_U * Zr[i] + (double)(nvr + 64) * 0x1p-1074;
            skip[i] = !(nvr > 0 && !__shfl(dom | unc, 4 * g + i, 64));
            const bool zok = Zr[i] > 2.0 * eZr[i] && isfinite(Zr[i]);
            rz[i] = zok ? 1.0 / Zr[i] : 0.0;
            rze[i] = zok ? 1.0 / (Zr[i] - eZr[i]) : 0.0;
            live[i] = !skip[i] && zok;
        }
        // output offsets of this lane's 4 rows (channel j of its first channel tile)
        int64_t orow[4];
        bool ovalid[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int lri = rbk * RPB + rg * 16 + 4 * g + i;
            ovalid[i] = lri < P.r_seg;
            const int lrv = ovalid[i] ? lri : 0;
            const int hq = hk * P.grp + lrv % P.grp;
            orow[i] = b * P.g.o_seq_stride + (int64_t)(lrv / P.grp) * P.g.o_tok_stride +
                      (int64_t)hq * P.g.o_head_stride + 16 * NCT * hh + j;
        }
        auto store_out = [&](int i, int cc, uint32_t bits) __attribute__((always_inline)) {
            if (P.out_fp32) ((uint32_t*)P.out)[orow[i] + 16 * cc] = bits;
            else ((uint16_t*)P.out)[orow[i] + 16 * cc] = (uint16_t)bits;
        };
        // every entry first tries the normal-range rounding (a few integer operations, no
        // branches); the entries it cannot decide go through LDS (the K and V buffers are idle:
        // no DMA is in flight) to one rolled loop of the general test
        double2* const qd = (double2*)smem + tid;  // entry e at qd[64 NWB e]
        uint32_t slow = 0;
        tick(11);
        const double omit = (double)ep_tiles * 0x1p20;
#pragma unroll
        for (int cc = 0; cc < NCT; ++cc) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                double en;
                const double nn = epoch_sum(cc, i, fr[i], omit, &en) + prev[4 * cc + i].x;
                en += prev[4 * cc + i].y;
                en += fabs(nn) * 0x1p-52;
                const double q = nn * rz[i];
                double delta = (en * (1.0 + 0x1p-40) + fabs(q) * eZr[i]) * rze[i] * (1.0 + 0x1p-40) +
                               fabs(q) * 0x1p-51 + 0x1p-1070;
                if (!isfinite(q) || !isfinite(delta) || !live[i]) delta = __builtin_inf();
                uint32_t bits = 0;
                const bool ok = !skip[i] && certify_round_normal(q, delta, P.out_fp32, &bits);
                if (ok && ovalid[i]) store_out(i, cc, bits);
                if (!skip[i] && !ok) {
                    slow |= 1u << (4 * cc + i);
                    qd[64 * NWB * (4 * cc + i)] = make_double2(q, delta);
                }
            }
        }
        tick(12);
        if (slow) {
#pragma unroll 1
            for (int e = 0; e < 4 * NCT; ++e) {
                if (!((slow >> e) & 1)) continue;
                const int cc = e >> 2, i = e & 3;
                const double2 v = qd[64 * NWB * e];
                uint32_t bits = 0;
                if (!certify_round_general(v.x, v.y, P.out_fp32, &bits)) {
                    failbits |= 1u << (8 * i + cc);
                    continue;
                }
                if (ovalid[i]) store_out(i, cc, bits);
            }
        }
    }
    tick(13);
    flush_timers(nt);
    if (P.stats) {
        const int st5 = wave_sum_i(nunc_s), st6 = wave_sum_i(nunc_w), st8 = wave_sum_i(nslow);
        if (lane == 0) {
            if (st5) atomicAdd((unsigned long long*)&P.stats[5], (unsigned long long)st5);
            if (st6) atomicAdd((unsigned long long*)&P.stats[6], (unsigned long long)st6);
            if (st8) atomicAdd((unsigned long long*)&P.stats[8], (unsigned long long)st8);
            if (nfold) atomicAdd((unsigned long long*)&P.stats[11], (unsigned long long)nfold);
            if (ncold) atomicAdd((unsigned long long*)&P.stats[12], (unsigned long long)ncold);
        }
    }
    if (nt == 0) {
        // no key visible to any row of the block: every row is empty (+0) or a q domain error
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
        pf_bar();  // sX reuse
        sX[w * 64 + lane].a = (int)fb;
        pf_bar();
#pragma unroll
        for (int o = 1; o < SPLIT; ++o) fb |= (uint32_t)sX[(rg * SPLIT + (hh + o) % SPLIT) * 64 + lane].a;
        failbits = fb;
    }
    int c_rows = 0, c_flag = 0, c_dom = 0, c_fin = 0;  // this lane's rows, added per wave below
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
            ++c_rows;
            c_flag += flag ? 1 : 0;
            c_dom += flag == 2 ? 1 : 0;
            c_fin += fin ? 1 : 0;
        }
    }
    // one atomic per counter and wave (same-address atomics per row would serialise)
    if (P.stats && hh == 0) {
        c_rows = wave_sum_i(c_rows);
        c_flag = wave_sum_i(c_flag);
        c_dom = wave_sum_i(c_dom);
        c_fin = wave_sum_i(c_fin);
        if (lane == 0) {
            if (c_rows) {
                atomicAdd((unsigned long long*)&P.stats[0], (unsigned long long)c_rows);
                atomicAdd((unsigned long long*)&P.stats[10], (unsigned long long)c_rows);
            }
            if (c_flag) atomicAdd((unsigned long long*)&P.stats[1], (unsigned long long)c_flag);
            if (c_dom) atomicAdd((unsigned long long*)&P.stats[4], (unsigned long long)c_dom);
            if (c_fin) atomicAdd((unsigned long long*)&P.stats[7], (unsigned long long)c_fin);
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Merge of the key splits' partials (pf_nsplit > 1) and the certified final rounding, one block of
// 128 threads per row (thread = channel). Per split s with keys: Z_s and N_s in units 2^base_s with
// bounds (nv_s + 8) u' Z_s + (nv_s + 64) 2^-1074 (the sums of the split's weights, as the kernel's
// own epilogue bounds them) and en_s. Rescaled to the largest base B by exact powers of two (an
// underflowing rescale loses at most 2^-1074 per term, added), then summed: ns - 1 more roundings
// of at most u of the sum of magnitudes. q = N RN(1/Z) and its radius as in ea_pf_main's epilogue,
// then certify_round; rows that fail go to the tier-2 work list.
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(128) ea_pf_combine(Params P) {
    const int64_t row = blockIdx.x;
    const int c = threadIdx.x;
    const int ns = P.pf_nsplit;
    const PfPart* const parts = (const PfPart*)P.pf_part;
    const double2* const ent = (const double2*)(parts + (int64_t)ns * P.rows);
    int B = INT_MIN, nv = 0, fl = 0;
    for (int s = 0; s < ns; ++s) {
        const PfPart pr = parts[(int64_t)s * P.rows + row];
        fl |= pr.fl;
        if (pr.nv > 0) {
            B = max(B, pr.base);
            nv += pr.nv;
        }
    }
    uint32_t bits = 0;
    bool fin = false;
    if (nv > 0 && !fl) {
        double z = 0.0, ezs = 0.0, nn = 0.0, an = 0.0, en = 0.0;
        for (int s = 0; s < ns; ++s) {
            const PfPart pr = parts[(int64_t)s * P.rows + row];
            if (pr.nv <= 0) continue;
            const int dsh = max(pr.base - B, -1100);
            const double zs = ldexp(pr.z, dsh);
            z += zs;
            ezs += (double)(pr.nv + 8) * PF_U * zs + (double)(pr.nv + 65) * 0x1p-1074;
            const double2 e = ent[((int64_t)s * P.rows + row) * 128 + c];
            const double v = ldexp(e.x, dsh);
            nn += v;
            an += fabs(v);
            en += ldexp(e.y, dsh) + 0x1p-1074;
        }
        // the merge's own roundings (ns - 1 additions each for Z and N, sums of positive bounds
        // rounded up by the (1 + 2^-40) factors)
        const double eZ = (ezs + (double)ns * PF_U * z) * (1.0 + 0x1p-40);
        en = (en + (double)ns * 0x1p-52 * an) * (1.0 + 0x1p-40);
        const bool zok = z > 2.0 * eZ && isfinite(z);
        const double rz = zok ? 1.0 / z : 0.0, rze = zok ? 1.0 / (z - eZ) : 0.0;
        const double q = nn * rz;
        double delta = (en * (1.0 + 0x1p-40) + fabs(q) * eZ) * rze * (1.0 + 0x1p-40) + fabs(q) * 0x1p-51 + 0x1p-1070;
        if (!isfinite(q) || !isfinite(delta) || !zok) delta = __builtin_inf();
        fin = !certify_round(q, delta, P.out_fp32, &bits);
        if (fin) bits = 0;
    }
    const bool anyfin = __syncthreads_or(fin) != 0;  // every thread reaches this barrier
    const int flag = (fl & 1) ? 2 : (((fl & 2) || anyfin) ? 1 : 0);
    const int Hq = P.g.num_q_heads, T = P.g.num_tokens;
    const int64_t b = row / ((int64_t)T * Hq);
    const int t = (int)((row / Hq) % T), hq = (int)(row % Hq);
    const int64_t o = b * P.g.o_seq_stride + (int64_t)t * P.g.o_tok_stride + (int64_t)hq * P.g.o_head_stride + c;
    if (flag) bits = 0;
    if (c < P.g.head_dim_v) {
        if (P.out_fp32) ((uint32_t*)P.out)[o] = bits;
        else ((uint16_t*)P.out)[o] = (uint16_t)bits;
    }
    if (c == 0) {
        P.flags[row] = (uint8_t)flag;
        if (flag == 1) {
            const int slot = atomicAdd(P.wl_cnt, 1);
            P.wl[slot] = (int32_t)row;
        }
        if (P.stats && flag) {
            atomicAdd((unsigned long long*)&P.stats[1], 1ull);
            if (flag == 2) atomicAdd((unsigned long long*)&P.stats[4], 1ull);
            if (flag == 1 && !(fl & 2)) atomicAdd((unsigned long long*)&P.stats[7], 1ull);
        }
    }
}

namespace {
// kernel shape: 32 rows per block; 8 waves (2 row groups x 4 waves, 2 waves per SIMD, 256
// registers each) by default, ea_options.prefill_waves = 4 selects 4 waves (2 x 2, 1 wave per SIMD)
constexpr int PF_RPB = 32;
}  // namespace

int ea::ea_prefill_eligible(const ea_geometry& g, int grp, int kernel, int* ntiles, int* nrb) {
    if (kernel == EA_KERNEL_DECODE || kernel == EA_KERNEL_GENERAL) return 0;
    const bool force = kernel == EA_KERNEL_PREFILL;
    if (g.head_dim != 128 || g.head_dim_v != 128) return 0;
    const int64_t r_seg = (int64_t)g.num_tokens * grp;
    // Rows of one (sequence, KV head) that fill a 32-row block (64 tokens, or fewer tokens with a
    // wider GQA group: speculative trees, chunked prefill) read each K/V tile once here, against
    // once per 1-2 rows in the decode kernel (C4: 0.82 ms here, 2.57 ms there with 4-row blocks)
    // Segments of 24-31 rows (verification of 12-15 draft tokens at GQA 2) come here too when
    // there is enough work: measured on MI355X against the decode kernel (2-row blocks, a
    // segment's row blocks on one XCD; contiguous K/V, graph replays), the int8 kernel is 14-45%
    // faster at 24 rows with 8K+ keys on 16+ segments or 32K+ keys on any; at 16 rows the decode
    // kernel is as fast or faster everywhere measured (up to 1.9x at 2K keys, within 3% at 64
    // segments of 32K keys).
    const int64_t nseg = (int64_t)g.num_seqs * g.num_kv_heads;
    const bool mid = r_seg >= 24 && g.max_seq_len >= 8192 && (nseg >= 16 || g.max_seq_len >= 32768);
    if (!force && g.num_tokens < 64 && r_seg < PF_RPB && !mid) return 0;
    if (r_seg >= (1 << 30) || (int64_t)g.max_seq_len + 64 >= (1 << 30)) return 0;
    const int rpb = PF_RPB;
    *ntiles = (g.max_seq_len + 63) / 64;
    *nrb = (int)((r_seg + rpb - 1) / rpb);
    return 1;
}

int ea::ea_launch_prefill(const Params& P, hipStream_t st) {
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    std::call_once(once, [] {
        const void* fns[4] = {(const void*)ea_pf_main<4, false>, (const void*)ea_pf_main<4, true>,
                              (const void*)ea_pf_main<8, false>, (const void*)ea_pf_main<8, true>};
        for (const void* f : fns)
            if (attr_err == hipSuccess)
                attr_err = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, PF_LDS);
    });
    if (attr_err != hipSuccess) return -100 - (int)attr_err;
    Params Pc = P;
    hipLaunchKernelGGL(ea_pf_qslice, dim3((unsigned)((P.rows + 15) / 16)), dim3(256), 0, st, Pc);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return -100 - (int)e;
    if (P.nseg > 0 && P.pf_ntiles > 0 && !P.pf_kv_cached) {
        hipLaunchKernelGGL(ea_pf_kvslice, dim3((unsigned)(P.nseg * P.pf_ntiles)), dim3(256), 0, st, Pc);
        e = hipGetLastError();
        if (e != hipSuccess) return -100 - (int)e;
    }
    return 0;
}

int ea::ea_launch_kv_digits(const Params& P, hipStream_t st) {
    if (P.nseg <= 0 || P.kvd_span <= 0) return 0;
    Params Pc = P;
    hipLaunchKernelGGL(ea_pf_kvslice, dim3((unsigned)(P.nseg * P.kvd_span)), dim3(256), 0, st, Pc);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : -100 - (int)e;
}

int ea::ea_launch_prefill_main(const Params& P, hipStream_t st) {
    Params Pc = P;
    if (P.nseg > 0 && P.pf_nrb > 0) {
        const dim3 grid((unsigned)(P.nseg * P.pf_nrb * P.pf_nsplit));
        if (P.pf_waves != 4) {
            if (P.timers) hipLaunchKernelGGL((ea_pf_main<8, true>), grid, dim3(512), PF_LDS, st, Pc);
            else hipLaunchKernelGGL((ea_pf_main<8, false>), grid, dim3(512), PF_LDS, st, Pc);
        } else {
            if (P.timers) hipLaunchKernelGGL((ea_pf_main<4, true>), grid, dim3(256), PF_LDS, st, Pc);
            else hipLaunchKernelGGL((ea_pf_main<4, false>), grid, dim3(256), PF_LDS, st, Pc);
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return -100 - (int)e;
    }
    return 0;
}

int ea::ea_launch_prefill_combine(const Params& P, hipStream_t st) {
    if (P.pf_nsplit <= 1 || P.rows == 0) return 0;
    Params Pc = P;
    hipLaunchKernelGGL(ea_pf_combine, dim3((unsigned)P.rows), dim3(128), 0, st, Pc);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : -100 - (int)e;
}
