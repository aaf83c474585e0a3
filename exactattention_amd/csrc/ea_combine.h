// Merge of the KV-split partials of one row and the certified final rounding (one wave per row;
// the combine kernel in ea_hip.hip).
#pragma once
#include "ea_params.h"

namespace ea {

// Returns the row's stats events, the same in every lane: bit 0 the row was merged (stats[0]),
// bit 1 it is flagged (stats[1]), bit 2 only its final rounding failed (stats[7]). The caller
// adds them up per block.
__device__ inline int combine_row(const Params& P, int64_t row, int lane) {
    const int dv = P.g.head_dim_v;
    const int Hq = P.g.num_q_heads, T = P.g.num_tokens;
    const int64_t b = row / ((int64_t)T * Hq);
    const int t = (int)((row / Hq) % T), hq = (int)(row % Hq);
    const int hk = hq / P.grp, gi = hq % P.grp;
    const int seg = (int)(b * P.g.num_kv_heads + hk);
    const int lr = t * P.grp + gi;
    const int rbk = lr / P.rb;
    // partials to merge: every split, or with the decode kernel's equal-share plan the pieces of
    // this row's unit (slots 0 .. npieces - 1; none for a unit without keys). The error bounds
    // below count nsb = nsplit merged terms either way (at least the number merged).
    const int nsb = P.nsplit;
    int ns = nsb;
    if (P.dq_stream) {
        const int u = seg * P.nrb + rbk, share = P.dq_plan[1];
        const int su = P.dq_plan[2 + u], tu = P.dq_plan[3 + u] - su;
        ns = tu > 0 ? (su + tu - 1) / share - su / share + 1 : 0;
    }
    const int J = (ns + 63) / 64;  // slabs of 64 splits: split 64 j + lane is this lane's in slab j

    // slab 0 may follow the caller's merge order: lane i holds split merge_order[i] when it is a
    // permutation of [0, ns) (ns <= 64); the sums below come from wave reductions, and any
    // summation order gives the same certified bits, so the order fixes only which lane loads what
    int si = lane;
    bool mo_ok = P.merge_order != nullptr && ns <= 64 && !P.dq_stream;
    if (mo_ok) {
        const int m = lane < ns ? P.merge_order[lane] : 0;
        const uint64_t bit = (lane < ns && m >= 0 && m < ns) ? (1ull << m) : 0ull;
        uint64_t seen = bit;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) seen |= __shfl_xor(seen, o, 64);
        mo_ok = seen == (ns == 64 ? ~0ull : ((1ull << ns) - 1));
        if (mo_ok) si = m;
    }
    // up to 8 splits in index order: every channel partial of both lane channels is requested
    // now, in the same round as the split scalars (one load latency per row instead of three);
    // splits that turn out empty are dropped by selects below
    const bool pre = ns <= 8 && !mo_ok && dv <= 128;
    double pfn[2][8];
    float pfv[2][8];
    if (pre) {
#pragma unroll
        for (int ci = 0; ci < 2; ++ci)
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int c = lane + 64 * ci;
                const bool in = k < ns && c < dv;
                const int64_t o = (int64_t)k * P.rows + row;
                pfn[ci][k] = in ? P.pN[o * dv + c] : 0.0;
                pfv[ci][k] = in ? P.pV[(((int64_t)k * P.nseg + seg) * P.nrb + rbk) * dv + c] : 0.0f;
            }
    }
    // the scalars (visible keys n, exponent r, Z) of this lane's split in slab j
    auto load_split = [&](int j, int* n, int* r, double* z) __attribute__((always_inline)) {
        const int i = 64 * j + lane;
        *n = 0;
        *r = INT_MIN;
        *z = 0.0;
        if (i < ns) {
            const int64_t o = (int64_t)(j == 0 ? si : i) * P.rows + row;
            *n = P.pn[o];
            *r = P.pR[o];
            *z = P.pZ[o];
        }
    };
    int n0, r0;
    double z0;
    load_split(0, &n0, &r0, &z0);
    int bad_l = n0 < 0, R_l = n0 > 0 ? r0 : INT_MIN;
    for (int j = 1; j < J; ++j) {
        int n, r;
        double z;
        load_split(j, &n, &r, &z);
        bad_l |= n < 0;
        if (n > 0) R_l = max(R_l, r);
    }
    const bool qbad = P.qinfo[row * 5 + 4] != 0;
    int flag = (__ballot(bad_l) != 0 || qbad) ? 1 : 0;
    const int R = wave_max_i(R_l);
    uint16_t* o16 = (uint16_t*)P.out;
    uint32_t* o32 = (uint32_t*)P.out;
    const int64_t obase = b * P.g.o_seq_stride + (int64_t)t * P.g.o_tok_stride + (int64_t)hq * P.g.o_head_stride;
    if (!flag && R == INT_MIN) {
        // no visible key: the output is +0 (docs/SPEC.md step 5, empty set)
        for (int c = lane; c < dv; c += 64) {
            if (P.out_fp32) o32[obase + c] = 0;
            else o16[obase + c] = 0;
        }
        if (lane == 0) P.flags[row] = 0;
        return 0;
    }
    const double up = 0x1p-53 * (1.0 + 0x1p-28);
    // the rounding depth inside one partial: n + 4, capped at 16 T + 6 for the decode kernel's
    // partials of at most T tiles (its lane chains hold 16 keys per tile)
    int64_t dcap = INT64_MAX;
    if (P.pv_tiles > 0) dcap = 16 * (int64_t)(P.dq_stream ? P.dq_plan[1] : P.pv_tiles) + 6;
    auto shift_of = [&](int n, int r) __attribute__((always_inline)) { return (n > 0 && R != INT_MIN) ? r - R : 0; };
    // Z and the bound's weight A = sum_s 2^(R_s - R) Zhat_s (D_s + nsplit), D_s = min(n_s + 4, dcap)
    double Z = 0.0, A = 0.0;
    int nterm = 0, far = 0;
    auto add_z = [&](int n, int r, double z) __attribute__((always_inline)) {
        const int dsh = shift_of(n, r);
        far |= (n > 0 && dsh < -900) ? 1 : 0;
        const double zs = n > 0 ? ldexp(z, max(dsh, -1000)) : 0.0;
        Z += zs;
        A += zs * (double)(min((int64_t)n + 4, dcap) + nsb);
        nterm += n > 0 ? n : 0;
    };
    add_z(n0, r0, z0);
    for (int j = 1; j < J; ++j) {
        int n, r;
        double z;
        load_split(j, &n, &r, &z);
        add_z(n, r, z);
    }
    if (__ballot(far) != 0) flag = 1;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        Z += __shfl_xor(Z, o, 64);
        A += __shfl_xor(A, o, 64);
        nterm += __shfl_xor(nterm, o, 64);
    }
    const double tiny = (double)(nterm + 64 * nsb + 64) * 0x1p-1074;
    const double eZ = A * up + tiny;
    if (!(Z > 2.0 * eZ) || !isfinite(Z)) flag = 1;
    bool ok = !flag;
    // certified rounding of channel c from its merged sum N and bound vmaxf on |v|
    auto finish = [&](int c, double N, float vmaxf) __attribute__((always_inline)) {
        uint32_t bits = 0;
        const double eN = A * up * (double)vmaxf + tiny;
        const double q = N / Z;
        const double aq = fabs(q);
        const double delta = (eN + aq * eZ) / (Z - eZ) * (1.0 + 0x1p-40) + aq * 0x1p-51 + 0x1p-1070;
        if (!isfinite(q) || !isfinite(delta) || !certify_round(q, delta, P.out_fp32, &bits)) ok = false;
        return bits;
    };
    const int dsh0 = shift_of(n0, r0);
    if (pre) {
        int nk[8], shk[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            nk[k] = __shfl(n0, k, 64);
            shk[k] = __shfl(dsh0, k, 64);
        }
#pragma unroll
        for (int ci = 0; ci < 2; ++ci) {
            const int c = lane + 64 * ci;
            if (c >= dv) continue;
            uint32_t bits = 0;
            if (!flag) {
                double N = 0.0;
                float vmaxf = 0.0f;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const bool use = k < ns && nk[k] > 0;
                    N += use ? ldexp(pfn[ci][k], max(shk[k], -1000)) : 0.0;
                    const float vm = use ? pfv[ci][k] : 0.0f;
                    vmaxf = fmaxf(vmaxf, vm);
                    if (!(vm <= 3.4028235e38f)) vmaxf = __builtin_inff();
                }
                bits = finish(c, N, vmaxf);
            }
            if (P.out_fp32) o32[obase + c] = bits;
            else o16[obase + c] = (uint16_t)bits;
        }
    } else {
        // per slab, both lane channels of 16 splits requested per round: a row of 32 splits waits
        // for 2 load latencies, of 64 for 4, and each further slab adds one for its scalars
        double N[2] = {0.0, 0.0};
        float vmaxf[2] = {0.0f, 0.0f};
        if (!flag) {
            for (int j = 0; j < J; ++j) {
                int sj = si, nj = n0, dj = dsh0;
                if (j > 0) {
                    int r;
                    double z;
                    load_split(j, &nj, &r, &z);
                    sj = 64 * j + lane;
                    dj = shift_of(nj, r);
                }
                const int cnt = min(64, ns - 64 * j);
                for (int i0 = 0; i0 < cnt; i0 += 16) {
                    double pn[2][16];
                    float pv[2][16];
                    int sh[16];
#pragma unroll
                    for (int k = 0; k < 16; ++k) {
                        const int i = i0 + k;
                        const int s = __shfl(sj, i & 63, 64), n = __shfl(nj, i & 63, 64);
                        sh[k] = __shfl(dj, i & 63, 64);
                        const bool use = i < cnt && n > 0;
                        const int64_t o = (int64_t)s * P.rows + row;
#pragma unroll
                        for (int ci = 0; ci < 2; ++ci) {
                            const int c = lane + 64 * ci;
                            const bool in = use && c < dv;
                            pn[ci][k] = in ? P.pN[o * dv + c] : 0.0;
                            pv[ci][k] = in ? P.pV[(((int64_t)s * P.nseg + seg) * P.nrb + rbk) * dv + c] : 0.0f;
                        }
                    }
#pragma unroll
                    for (int k = 0; k < 16; ++k)
#pragma unroll
                        for (int ci = 0; ci < 2; ++ci) {
                            N[ci] += ldexp(pn[ci][k], max(sh[k], -1000));
                            vmaxf[ci] = fmaxf(vmaxf[ci], pv[ci][k]);
                            if (!(pv[ci][k] <= 3.4028235e38f)) vmaxf[ci] = __builtin_inff();
                        }
                }
            }
        }
#pragma unroll
        for (int ci = 0; ci < 2; ++ci) {
            const int c = lane + 64 * ci;
            if (c >= dv) continue;
            const uint32_t bits = flag ? 0u : finish(c, N[ci], vmaxf[ci]);
            if (P.out_fp32) o32[obase + c] = bits;
            else o16[obase + c] = (uint16_t)bits;
        }
    }
    const int bad = wave_max_i(ok ? 0 : 1);
    if (lane == 0) {
        P.flags[row] = bad ? 1 : 0;
        if (bad) {
            const int slot = atomicAdd(P.wl_cnt, 1);
            P.wl[slot] = (int32_t)row;
        }
    }
    return 1 | (bad ? 2 : 0) | ((bad && !flag) ? 4 : 0);
}

}  // namespace ea
