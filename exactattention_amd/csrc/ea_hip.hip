// Certified split-KV ExactAttention for AMD Instinct MI355X (gfx950): kernels and C ABI.
//
// One step is four launches on the caller's stream, with fixed grids and no memsets:
//   ea_prep      q rows -> fp64 + exponent ranges; clears the tier-2 work counter (the decode
//                kernel on uniform splits does both itself, and the step is three launches)
//   ea_split     tier 1: per (segment, row block, KV split) an fp64 pass over 64-key tiles:
//                exact scores (checked), certified logits and weights, P.V partials with
//                rigorous error bounds. Writes one partial per (split, row).
//   ea_combine   merges the split partials in the caller's order and certifies RN(N/Z) per
//                channel; appends rows it cannot certify to the tier-2 work list
//   ea_tier2     per listed row: 128-bit windowed scores, 128-bit exp2 enclosure, 128-bit
//                fixed-point Z and N with counted truncation, exact final rounding
// Reference behaviour: src/exactattn/triton_kernels.py:1324-1519 (split, combine, tier 2,
// host fallback) and docs/SPEC.md (the definition the bits must equal).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "../../include/exactattn_hip.h"
#include "ea_device.h"
#include "ea_params.h"
#include "ea_combine.h"
#include "ea_exact.h"

using namespace ea;

// ------------------------------------------------------------------------------------------------
// Kernel 1: q rows to fp64 plus per-32-dim-block exponent ranges and |q| sums (prep_row_store),
// one wave per row; block 0 clears the tier-2 work list, and on the decode kernel's stream plan an
// extra last block writes that plan.
// ------------------------------------------------------------------------------------------------
// The decode kernel's equal-share plan (Params::dq_*), by one 256-thread block: per unit its tile
// count (up to unit_kend, at most dq_max_tiles), the exclusive prefix sums S_u with S_units = W, the
// share max(ceil(W / dq_blocks), dq_min_share), and per block g its first piece as one record
// (unit u, S_u, S_(u+1), share): the unit holding tile g share is the u with
// S_u <= g share < S_(u+1), so the blocks g in [ceil(S_u / share), ceil(S_(u+1) / share)) start in
// unit u and each is written by that unit's thread. Blocks past W get u = units. Every entry the
// decode kernel and the combine read is written here.
__device__ void dq_plan_block(const Params& P) {
    __shared__ int s_scan[2][256];
    __shared__ int s_share;
    const int tid = threadIdx.x, U = P.dq_units, G = P.dq_blocks;
    int32_t* plan = P.dq_plan;
    int32_t* Su = plan + 2;
    int4* brec = (int4*)(plan + P.dq_rec_off);
    const int per = (U + 255) / 256;
    const int u0 = min(tid * per, U), u1 = min(u0 + per, U);
    auto tiles = [&](int u) { return min((unit_kend(P, u / P.nrb, u % P.nrb) + 63) >> 6, P.dq_max_tiles); };
    int sum = 0;
    for (int u = u0; u < u1; ++u) sum += tiles(u);
    // inclusive scan of the 256 chunk sums (Hillis-Steele, ping-pong)
    int cur = 0;
    s_scan[0][tid] = sum;
    __syncthreads();
    for (int o = 1; o < 256; o <<= 1) {
        const int x = s_scan[cur][tid] + (tid >= o ? s_scan[cur][tid - o] : 0);
        s_scan[cur ^ 1][tid] = x;
        cur ^= 1;
        __syncthreads();
    }
    const int W = s_scan[cur][255];
    if (tid == 0) {
        const int share = max(max((W + G - 1) / G, P.dq_min_share), 1);
        s_share = share;
        plan[0] = W;
        plan[1] = share;
        Su[U] = W;
        if (P.stats) atomicAdd((unsigned long long*)&P.stats[15], 1ull);
    }
    __syncthreads();
    const int share = s_share;
    int run = s_scan[cur][tid] - sum;  // exclusive prefix of this thread's chunk
    for (int u = u0; u < u1; ++u) {
        const int t = tiles(u);
        Su[u] = run;
        for (int g = (run + share - 1) / share; g * share < run + t && g < G; ++g)
            brec[g] = make_int4(u, run, run + t, share);
        run += t;
    }
    const int nb = (W + share - 1) / share;  // blocks with a share: [0, nb)
    for (int g = nb + tid; g < G; g += 256) brec[g] = make_int4(U, W, W, share);
}

__global__ void __launch_bounds__(256) ea_prep(Params P) {
    if (blockIdx.x == 0 && threadIdx.x <= EA_T2_BLOCKS) P.wl_cnt[threadIdx.x] = 0;
    if (P.dq_stream && blockIdx.x == gridDim.x - 1) {
        dq_plan_block(P);  // the extra last block
        return;
    }
    int lane = threadIdx.x & 63;
    int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= P.rows) return;
    int Hq = P.g.num_q_heads, T = P.g.num_tokens, d = P.g.head_dim;
    int64_t b = row / ((int64_t)T * Hq);
    int t = (int)((row / Hq) % T), hq = (int)(row % Hq);
    const uint16_t* qr = P.q + b * P.g.q_seq_stride + (int64_t)t * P.g.q_tok_stride + (int64_t)hq * P.g.q_head_stride;
    // dims past d enter as +0 (stored as 0.0, no exponent, no flag)
    const uint32_t x0 = 2 * lane < d ? qr[2 * lane] : 0u, x1 = 2 * lane + 1 < d ? qr[2 * lane + 1] : 0u;
    (void)prep_row_store(P, row, lane, x0, x1);
}

// ------------------------------------------------------------------------------------------------
// Kernel 2: tier-1 split kernel, templated on the rows per block (1, 2 or 4).
// Block = 4 waves over one (segment, row block, KV split); 64-key tiles, 2 barriers per tile:
//   [1] K(i) is in LDS (double-buffered, 16-byte chunks XOR-swizzled so per-key reads are
//       conflict-free).
//   S   wave w, lane = key: fp64 FMA chains over dims [32w, 32w+32) in 8-dim steps, q read
//       through the constant address space (scalar loads, SGPR operands). The block's sum is
//       exact when (FQmax-FQmin') + (FKmax-FKmin') <= 32 over those dims: every partial sum is
//       then a multiple of the smallest product lsb and below 2^53 of it.
//   [2] the 4 block sums of every (row, key) are in LDS.
//   B   wave w, lanes = (row r, key 16w + l): the 4 exact block sums added with TwoSum
//       (error-free), so s lies in [S + sig - 3u E, S + sig + 3u E], E the sum of the TwoSum errors
//       (0 when the fp64 sum is exact); pairs whose blocks were not certified exact are redone
//       product by product. Certified t = RN32(alpha s); w = RN24(2^t) (fp64 tables; 128-bit
//       enclosure when undecided). Each wave keeps its own running reference exponent per row.
//   P   wave w: channels 2l, 2l+1 over its 16 keys from registers (the V row of a wave-uniform key:
//       one 256-byte coalesced load, page lookup on the scalar unit), FMA-fused exact products.
//       Then V(i+1) is requested and K(i+1) stored to the other LDS buffer.
// The epilogue merges the 4 wave partials of each row (exact power-of-two rescale, 3 additions).
// ------------------------------------------------------------------------------------------------
struct SplitSmem {
    uint4 K[2][EA_TILE * 16];            // 32 KB, swizzled chunks; the epilogue reuses it
    double T1[256], T2[256];             // 4 KB
    double sc[4][EA_MAXRB][EA_TILE];     // 8 KB block sums
    uint32_t fm[4][EA_TILE];             // 1 KB: bit r = block sum of row r not certified exact
    double w[4][EA_MAXRB][16];           // 2 KB: each wave's weights of its 16 keys
    int32_t wR[4][EA_MAXRB];             // epilogue: per-wave reference exponents
    double wZ[4][EA_MAXRB];
    int32_t wn[4][EA_MAXRB];
    uint32_t vred[4][64];                // 1 KB
};

template <int RB, bool TIMERS>
__global__ void __launch_bounds__(EA_THREADS, 2) ea_split(Params P) {
    uint64_t tclk[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint64_t tprev = TIMERS ? __builtin_amdgcn_s_memtime() : 0;
    auto tick = [&](int ph) {
        if (TIMERS) {
            uint64_t t = __builtin_amdgcn_s_memtime();
            tclk[ph] += t - tprev;
            tprev = t;
        }
    };
    extern __shared__ __align__(16) unsigned char smem_raw[];
    SplitSmem& S = *reinterpret_cast<SplitSmem*>(smem_raw);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int d = P.g.head_dim, dv = P.g.head_dim_v;
    const int nchunk = d >> 3;   // 16-byte chunks per key row
    const int ndw = dv >> 1;     // dwords per value row

    const int item = blockIdx.x;
    const int seg = item / P.nrb, rbk = item % P.nrb;
    const int split = blockIdx.y;
    const int Hkv = P.g.num_kv_heads;
    const int64_t b = seg / Hkv;
    const int hk = seg % Hkv;
    const int row0 = rbk * P.rb;
    const int nrow = min(RB, P.r_seg - row0);

    for (int i = tid; i < 256; i += EA_THREADS) {
        S.T1[i] = u64_as_f64(EA_T1_BITS[i]);
        S.T2[i] = u64_as_f64(EA_T2_BITS[i]);
    }
    // rows of the block (a short block repeats its last row; repeats are never written)
    int64_t grow[RB];
    int64_t kend = 0;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        int lr = row0 + min(r, nrow - 1);
        int t = lr / P.grp, gi = lr % P.grp;
        grow[r] = row_index(P, b, t, hk * P.grp + gi);
        kend = max(kend, vis_end(P, b * P.g.num_tokens + t, b));
    }
    // B-phase role: lane -> (row br, key 16w + bk); lanes with br >= nrow only idle
    const int br = lane >> 4, bk = lane & 15;
    const bool brow_ok = br < nrow;
    int64_t my_grow = 0;
    int64_t my_kvl = 0, my_tb = 0;
    uint64_t my_tm = 0;
    if (brow_ok) {
        int lr = row0 + br;
        int t = lr / P.grp, gi = lr % P.grp;
        my_grow = row_index(P, b, t, hk * P.grp + gi);
        int64_t tok = b * P.g.num_tokens + t;
        my_kvl = P.kv_len[tok];
        if (P.tree_mask) {
            my_tm = P.tree_mask[tok];
            my_tb = P.tree_base[b];
        }
    }
    const int64_t slen = P.seq_len[b];
    if (kend > slen) kend = slen;
    const int64_t k0 = (int64_t)split * P.split_len;
    const int64_t k1 = min(k0 + (int64_t)P.split_len, kend);
    const int64_t pbase = (int64_t)split * P.rows;
    const int64_t bt_off = P.bt ? (P.bt_off ? P.bt_off[b] : b * (int64_t)P.g.block_table_stride) : 0;
    cint_t* bt4 = (cint_t*)P.bt;
    const int pmask = (1 << P.pshift) - 1;

    // exponent ranges of this wave's q block for each row (scalar loads)
    cint_t* qinfo4 = (cint_t*)P.qinfo;
    int qspread[RB];
    bool qzero[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        int32_t qi = qinfo4[grow[r] * 5 + w];
        qzero[r] = (qi == (int32_t)0x80000000);
        qspread[r] = ((qi >> 16) & 0x1FF) - (qi & 0xFFFF);
    }
    // per-lane (B role) row state; the flag and running exponent are uniform within a row's
    // 16 lanes
    int rflag = (brow_ok && qinfo4[my_grow * 5 + 4]) ? 1 : 0;
    int Rrun = INT_MIN;
    double zacc = 0.0;
    int nvis = 0;

    double acc[RB][2];
#pragma unroll
    for (int r = 0; r < RB; ++r) acc[r][0] = acc[r][1] = 0.0;
    uint32_t vmx = 0;  // packed max |v| magnitude bits, channels 2*lane, 2*lane+1

    // K loader role: key kt = tid/4, 64-byte quarter qq = tid%4 (chunks 4j + qq, j = 0..3)
    const int kt = tid >> 2, qq = tid & 3;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 kst[4];
    auto load_k = [&](int64_t n0) {
        int64_t n = n0 + kt;
        bool ok = n < k1;
        int64_t page = b, slot = n;
        if (ok && P.bt) {
            page = P.bt[bt_off + (n >> P.pshift)];
            slot = n & pmask;
        }
        const u32x4* kp = reinterpret_cast<const u32x4*>(P.k + page * P.g.k_page_stride + slot * P.g.k_slot_stride +
                                                         (int64_t)hk * P.g.k_head_stride);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int c = 4 * j + qq;
            u32x4 a = {0, 0, 0, 0};
            if (ok && c < nchunk) a = __builtin_nontemporal_load(kp + c);
            kst[j] = a;
        }
    };
    auto store_k = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int c = 4 * j + qq;
            S.K[buf][kt * 16 + (c ^ (kt & 15))] = make_uint4(kst[j].x, kst[j].y, kst[j].z, kst[j].w);
        }
    };
    // V loader role (wave w, keys 16w..16w+15 of the tile, dword `lane` of each row)
    uint32_t vr[16];
    auto load_v = [&](int64_t n0) {
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            int64_t n = n0 + 16 * w + kk;  // wave-uniform
            uint32_t val = 0;
            if (n < k1) {
                int64_t page = b, slot = n;
                if (P.bt) {
                    page = bt4[bt_off + (n >> P.pshift)];
                    slot = n & pmask;
                }
                const uint32_t* vp = reinterpret_cast<const uint32_t*>(
                    P.v + page * P.g.v_page_stride + slot * P.g.v_slot_stride + (int64_t)hk * P.g.v_head_stride);
                if (lane < ndw) val = __builtin_nontemporal_load(vp + lane);
            }
            vr[kk] = val;
        }
    };

    const int ntiles = (k1 > k0) ? (int)((k1 - k0 + EA_TILE - 1) / EA_TILE) : 0;
    if (ntiles > 0) {
        load_k(k0);
        load_v(k0);
        store_k(0);
        if (ntiles > 1) load_k(k0 + EA_TILE);
    }
    const int spread_lim = 32;

    tick(0);
    for (int it = 0; it < ntiles; ++it) {
        const int buf = it & 1;
        const int64_t n0 = k0 + (int64_t)it * EA_TILE;
        __syncthreads();  // [1] K(i) visible; every wave is past B(i-1)
        tick(1);

        // ---- S: dims [32w, 32w+32) of key `lane`, every row
        {
            // re-read q through the scalar cache every tile: hoisting 32*RB doubles out of the
            // loop would exceed the SGPR file and spill them to VGPR lanes
            uint64_t qaddr = (uint64_t)P.q64;
            asm volatile("" : "+s"(qaddr));
            cdouble_t* q4 = (cdouble_t*)qaddr;
            typedef unsigned short us2 __attribute__((ext_vector_type(2)));
            us2 mx = {0, 0}, mn = {0xFFFF, 0xFFFF};
            double a0[RB], a1[RB];
#pragma unroll
            for (int r = 0; r < RB; ++r) a0[r] = a1[r] = 0.0;
#pragma unroll 1
            for (int cc = 0; cc < 4; ++cc) {
                const int c = 4 * w + cc;
                uint4 kv = (c < nchunk) ? S.K[buf][lane * 16 + (c ^ (lane & 15))] : make_uint4(0, 0, 0, 0);
                uint32_t kd[4] = {kv.x, kv.y, kv.z, kv.w};
                double kf[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    us2 mv = __builtin_bit_cast(us2, kd[j] & 0x7FFF7FFFu);
                    mx = __builtin_elementwise_max(mx, mv);
                    mn = __builtin_elementwise_min(mn, mv - (us2){1, 1});
                    kf[2 * j] = bf16lo_f64(kd[j]);
                    kf[2 * j + 1] = bf16hi_f64(kd[j]);
                }
#pragma unroll
                for (int r = 0; r < RB; ++r) {
                    cdouble_t* qr = q4 + grow[r] * EA_MAXD + 8 * c;
#pragma unroll
                    for (int i = 0; i < 8; i += 2) {
                        a0[r] = __fma_rn(qr[i], kf[i], a0[r]);
                        a1[r] = __fma_rn(qr[i + 1], kf[i + 1], a1[r]);
                    }
                }
            }
            uint32_t magmax = max((uint32_t)mx.x, (uint32_t)mx.y);
            uint32_t magmin1 = min((uint32_t)mn.x, (uint32_t)mn.y);
            bool kzero = (magmax == 0);
            int kspread = (int)(magmax >> 7) - max((int)((magmin1 + 1) >> 7), 1);
            uint32_t fmask = 0;
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                S.sc[w][r][lane] = a0[r] + a1[r];
                bool exact = qzero[r] || kzero || (qspread[r] + kspread <= spread_lim);
                if (!exact) fmask |= 1u << r;
            }
            S.fm[w][lane] = fmask;
        }
        if (it + 1 < ntiles) store_k(buf ^ 1);  // K(i+1); buffer buf^1 was last read in S(i-1)
        if (it + 2 < ntiles) load_k(n0 + 2 * EA_TILE);
        tick(2);
        __syncthreads();  // [2]
        tick(3);

        // ---- B: lanes (row br, key 16w + bk)
        {
            const int key = 16 * w + bk;
            const int64_t n = n0 + key;
            const int64_t ti = n - my_tb;
            const bool vis = brow_ok && (n < k1) && (n < my_kvl || (ti >= 0 && ti < 64 && ((my_tm >> ti) & 1)));
            const int r = brow_ok ? br : 0;
            double x0 = S.sc[0][r][key], x1 = S.sc[1][r][key], x2 = S.sc[2][r][key], x3 = S.sc[3][r][key];
            bool slow = ((S.fm[0][key] | S.fm[1][key] | S.fm[2][key] | S.fm[3][key]) >> r) & 1;
            double ssum, sig, del;
            if (vis && slow) {
                // every product separately, TwoSum-accumulated: exact up to the rounding of the
                // error sum, bounded by 256 u E (E = sum of |TwoSum errors|, 2 roundings per add)
                cdouble_t* qr = (cdouble_t*)P.q64 + my_grow * EA_MAXD;
                double s = 0.0, es = 0.0, ea = 0.0;
                for (int c = 0; c < nchunk; ++c) {
                    uint4 kv = S.K[buf][key * 16 + (c ^ (key & 15))];
                    uint32_t wd[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        double e0, e1;
                        s = two_sum(s, qr[8 * c + 2 * j] * bf16lo_f64(wd[j]), &e0);
                        s = two_sum(s, qr[8 * c + 2 * j + 1] * bf16hi_f64(wd[j]), &e1);
                        es += e0 + e1;
                        ea += fabs(e0) + fabs(e1);
                    }
                }
                ssum = s;
                sig = es;
                del = ea * 0x1p-44;
            } else {
                double e1, e2, e3;
                double s = two_sum(x0, x1, &e1);
                s = two_sum(s, x2, &e2);
                s = two_sum(s, x3, &e3);
                ssum = s;
                sig = (e1 + e2) + e3;
                del = (fabs(e1) + fabs(e2) + fabs(e3)) * 0x1p-51;
            }
            int32_t M = 1 << 23, E = -23;
            int why = 0;  // 1 score not certified, 2 weight not certified
            if (vis && !rflag) {
                uint32_t tb = 0;
                int ls = (ssum == 0.0 && sig == 0.0 && del == 0.0) ? 1
                         : (isfinite(ssum) ? logit_cert(P.alpha, ssum, sig, del, &tb) : 3);
                if (ls == 2 || ls == 3) {
                    why = 1;  // overflow (tier 2 reports the domain error) or undecided
                } else if (ls == 0) {
                    int ws = weight_f64(tb, S.T1, S.T2, &M, &E);
                    if (ws) {
                        int32_t M2 = 0;
                        int64_t E2 = 0;
                        if (weight_wide(tb, &M2, &E2) == 0 && E2 > -(1LL << 30) && E2 < (1LL << 30)) {
                            M = M2;
                            E = (int32_t)E2;
                        } else {
                            why = 2;
                        }
                    }
                }
            }
            if (P.stats) {
                uint64_t b1 = __ballot(why == 1), b2 = __ballot(why == 2), b3 = __ballot(vis && slow);
                if (lane == 0 && b1) atomicAdd((unsigned long long*)&P.stats[5], (unsigned long long)__popcll(b1));
                if (lane == 0 && b2) atomicAdd((unsigned long long*)&P.stats[6], (unsigned long long)__popcll(b2));
                if (lane == 0 && b3) atomicAdd((unsigned long long*)&P.stats[8], (unsigned long long)__popcll(b3));
            }
            if (why) rflag = 1;
            // maxima over each row's 16 lanes (one DPP row each)
            rflag = row16_max(rflag);
            int tmax = row16_max(vis ? E + 23 : INT_MIN);
            int Rnew = max(Rrun, tmax);
            double sc = 1.0;
            if (Rrun != INT_MIN && Rnew != Rrun) {
                int dsh = Rrun - Rnew;
                if (dsh < -900) rflag = 1;
                sc = ldexp(1.0, max(dsh, -1000));
                zacc *= sc;
            }
            double om = 0.0;
            if (vis) {
                int de = E - Rnew;
                if (de < -1000) rflag = 1;
                om = ldexp((double)M, max(de, -1000));
            }
            if (rflag) om = 0.0;
            zacc += om;
            nvis += vis ? 1 : 0;
            Rrun = Rnew;
            if (brow_ok) S.w[w][br][bk] = om;
            // rescale this wave's accumulators by each row's factor (uniform per row)
#pragma unroll
            for (int rr = 0; rr < RB; ++rr) {
                double f = __shfl(sc, rr * 16, 64);
                if (f != 1.0) {
                    acc[rr][0] *= f;
                    acc[rr][1] *= f;
                }
            }
        }

        tick(4);
        // ---- P: channels 2*lane, 2*lane+1 over keys 16w .. 16w+15 (weights of this wave)
        {
            typedef unsigned short us2 __attribute__((ext_vector_type(2)));
            us2 vm = __builtin_bit_cast(us2, vmx);
#pragma unroll 2
            for (int kk = 0; kk < 16; kk += 2) {
                uint32_t vd0 = vr[kk], vd1 = vr[kk + 1];
                vm = __builtin_elementwise_max(vm, __builtin_bit_cast(us2, vd0 & 0x7FFF7FFFu));
                vm = __builtin_elementwise_max(vm, __builtin_bit_cast(us2, vd1 & 0x7FFF7FFFu));
                double v00 = bf16lo_f64(vd0), v01 = bf16hi_f64(vd0);
                double v10 = bf16lo_f64(vd1), v11 = bf16hi_f64(vd1);
#pragma unroll
                for (int r = 0; r < RB; ++r) {
                    double2 om = *reinterpret_cast<const double2*>(&S.w[w][r][kk]);
                    acc[r][0] = __fma_rn(om.x, v00, acc[r][0]);
                    acc[r][1] = __fma_rn(om.x, v01, acc[r][1]);
                    acc[r][0] = __fma_rn(om.y, v10, acc[r][0]);
                    acc[r][1] = __fma_rn(om.y, v11, acc[r][1]);
                }
            }
            vmx = __builtin_bit_cast(uint32_t, vm);
        }
        if (it + 1 < ntiles) load_v(n0 + EA_TILE);
        tick(5);
    }

    // ---- epilogue: merge the 4 wave partials of each row, write the split partial
    {
        // row scalars of this wave (lane 16 r holds row r's running exponent and flag)
        double z = zacc;
        int nv = nvis;
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) {  // sums within each 16-lane row
            z += __shfl_xor(z, o, 64);
            nv += __shfl_xor(nv, o, 64);
        }
        if (bk == 0 && br < RB) {
            S.wR[w][br] = rflag ? -0x7FFFFFFF : Rrun;  // INT_MIN = no key, -0x7FFFFFFF = flagged
            S.wZ[w][br] = z;
            S.wn[w][br] = nv;
        }
    }
    __syncthreads();
    double* red = reinterpret_cast<double*>(&S.K[0][0]);  // 4 * EA_MAXRB * 128 doubles = 16 KB
    if (lane < ndw) {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            red[((w * EA_MAXRB) + r) * 128 + 2 * lane] = acc[r][0];
            red[((w * EA_MAXRB) + r) * 128 + 2 * lane + 1] = acc[r][1];
        }
    }
    S.vred[w][lane] = vmx;
    __syncthreads();
    for (int x = tid; x < nrow * dv; x += EA_THREADS) {
        int r = x / dv, c = x % dv;
        int R = INT_MIN;
        bool fl = false;
        for (int ww = 0; ww < 4; ++ww) {
            int rw = S.wR[ww][r];
            if (rw == -0x7FFFFFFF) fl = true;
            else R = max(R, rw);
        }
        double s = 0.0, zs = 0.0;
        int nv = 0;
        for (int ww = 0; ww < 4; ++ww) {
            int rw = S.wR[ww][r];
            if (rw == INT_MIN || rw == -0x7FFFFFFF) continue;
            if (rw - R < -900) fl = true;
            s += ldexp(red[((ww * EA_MAXRB) + r) * 128 + c], max(rw - R, -1000));
            zs += ldexp(S.wZ[ww][r], max(rw - R, -1000));
            nv += S.wn[ww][r];
        }
        int lr = row0 + r;
        int t = lr / P.grp, gi = lr % P.grp;
        int64_t o = pbase + row_index(P, b, t, hk * P.grp + gi);
        P.pN[o * dv + c] = s;
        if (c == 0) {
            P.pR[o] = R;
            P.pZ[o] = zs;
            P.pn[o] = fl ? -1 : nv;
        }
    }
    for (int c = tid; c < dv; c += EA_THREADS) {
        uint32_t m = 0;
        for (int ww = 0; ww < 4; ++ww) {
            uint32_t a = S.vred[ww][c >> 1];
            m = max(m, (c & 1) ? (a >> 16) : (a & 0xFFFF));
        }
        // bf16 magnitude bits -> fp32 value (a NaN pattern keeps the row from certifying)
        P.pV[(((int64_t)split * P.nseg + seg) * P.nrb + rbk) * dv + c] = __uint_as_float(m << 16);
    }
    if (TIMERS) {
        tick(6);
        tclk[7] = (uint64_t)ntiles;
        if (lane == 0)
            for (int i = 0; i < 8; ++i) atomicAdd((unsigned long long*)&P.timers[i], (unsigned long long)tclk[i]);
    }
}

// ------------------------------------------------------------------------------------------------
// Kernel 3: combine. One wave per row. Merges the split partials in merge order, then the
// certified rounding per channel. Rows not certified go to the tier-2 work list.
// Error bound (u = 2^-53, relative weights w_j 2^-R of the split, n_s visible keys):
//   |Zhat_s - Z_s| <= D_s u' Z_s,  |Nhat_sc - N_sc| <= D_s u' Vmax_sc Z_s
// where D_s bounds the roundings on any term's path through the split's sums (FMA-fused exact
// products, u' = u (1 + 2^-28)). Any summation tree of n_s nonzero terms has at most n_s - 1
// rounding additions on a path (additions of exact zeros are exact), so D_s = n_s + 4 always
// holds. The d = 128 decode kernel's sums are shallower (pv_tiles > 0): each lane's P.V chain
// takes at most 16 keys of each of the partial's T tiles, then 2 additions merge the 4 key groups;
// each lane's Z chain takes one key per tile, then a 6-level wave sum. There
// D_s = min(n_s + 4, 16 T + 6), T the most tiles of one partial (split_len / 64, or the share of
// the equal-share plan). Merging adds depth nsplit, so with A = sum_s 2^(R_s - R) Zhat_s
// (D_s + nsplit):
//   eZ = u' A + tiny,  eN_c = u' A max_s Vmax_sc + tiny.
// ------------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(64) ea_combine(Params P) {
    // one row per 64-thread block: the merge is a chain of dependent loads, so it wants as many
    // rows in flight as the machine holds. stats[0] counts the step's rows once; the per-row
    // counters only move for flagged rows (rare), so they never serialise on one address.
    const int64_t row = blockIdx.x;
    if (row == 0 && threadIdx.x == 0 && P.stats) atomicAdd((unsigned long long*)&P.stats[0], (unsigned long long)P.rows);
    const int ev = combine_row(P, row, threadIdx.x);
    if (threadIdx.x == 0 && P.stats && (ev & 2)) {
        atomicAdd((unsigned long long*)&P.stats[1], 1ull);
        if (ev & 4) atomicAdd((unsigned long long*)&P.stats[7], 1ull);
    }
}

// ------------------------------------------------------------------------------------------------
// Kernel 4: tier 2. One block per listed row (grid-stride over the work list). 128-bit arithmetic
// throughout; the same certified structure as the reference's int128 CPU schedule
// (csrc/exact_attention_cpu.cpp:361-490 with acc_bits = 128), with a single tile per row.
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ i128 floor_shift128(i128 m, int64_t sh, int* lost) {
    if (sh >= 0) {
        *lost = 0;
        return m << sh;
    }
    int64_t s = -sh;
    if (s >= 127) {
        *lost = m != 0;
        return m < 0 ? (i128)-1 : (i128)0;
    }
    i128 v = m >> s;
    *lost = (v << s) != m;
    return v;
}

#define EA_T2_THREADS 512
#define EA_T2_WAVES (EA_T2_THREADS / 64)
struct T2Smem {
    double T1[256], T2[256];
    int32_t qm[EA_MAXD], qe[EA_MAXD];
    uint64_t red_hi[EA_T2_THREADS], red_lo[EA_T2_THREADS];
    int64_t red_i[EA_T2_THREADS];
    // per wave and channel: the N pass's partial maxima, then its 128-bit sums and lost counts
    int64_t nrw[EA_T2_WAVES][EA_MAXDV];
    uint64_t ahi[EA_T2_WAVES][EA_MAXDV], alo[EA_T2_WAVES][EA_MAXDV], aer[EA_T2_WAVES][EA_MAXDV];
    int32_t flag;
};

__device__ void block_reduce_i128(T2Smem& S, i128* v, uint64_t* err) {
    int tid = threadIdx.x;
    S.red_hi[tid] = (uint64_t)((u128)*v >> 64);
    S.red_lo[tid] = (uint64_t)(u128)*v;
    S.red_i[tid] = (int64_t)*err;
    __syncthreads();
    for (int s = EA_T2_THREADS / 2; s > 0; s >>= 1) {
        if (tid < s) {
            u128 a = ((u128)S.red_hi[tid] << 64) | S.red_lo[tid];
            u128 c = ((u128)S.red_hi[tid + s] << 64) | S.red_lo[tid + s];
            u128 x = a + c;
            S.red_hi[tid] = (uint64_t)(x >> 64);
            S.red_lo[tid] = (uint64_t)x;
            S.red_i[tid] += S.red_i[tid + s];
        }
        __syncthreads();
    }
    *v = (i128)(((u128)S.red_hi[0] << 64) | S.red_lo[0]);
    *err = (uint64_t)S.red_i[0];
    __syncthreads();
}

__device__ int block_max_i64(T2Smem& S, int64_t x, int64_t* out) {
    int tid = threadIdx.x;
    S.red_i[tid] = x;
    __syncthreads();
    for (int s = EA_T2_THREADS / 2; s > 0; s >>= 1) {
        if (tid < s) S.red_i[tid] = max(S.red_i[tid], S.red_i[tid + s]);
        __syncthreads();
    }
    *out = S.red_i[0];
    __syncthreads();
    return 0;
}

// One key chunk's share of a row that tier 2 splits over several blocks: the chunk's sums against
// its own window bases (R_b - F for Z, nr_c - F for channel c), each as a floor with a count of
// units lost to the floors.
struct T2Part {
    int64_t R;                 // max over the chunk's keys of E + 23 (INT64_MIN: no key)
    int32_t flag;              // 0, 1 (a logit or weight not certified), 2 (domain error)
    int32_t pad;
    uint64_t zhi, zlo, ze;     // Z_b in units 2^(R - F) and its lost count
    int64_t nr[EA_MAXDV];      // NR_c over the chunk (INT64_MIN: no nonzero V element)
    uint64_t nhi[EA_MAXDV], nlo[EA_MAXDV], ner[EA_MAXDV];  // N_c,b in units 2^(nr_c - F), lost count
};

// Rows are split into C key chunks when fewer rows are listed than there are blocks (C = blocks /
// rows, so one flagged row takes every block instead of one): block (row slot, chunk) computes the
// chunk's logits and weights and its Z and N sums, writes them as a T2Part, and the row's last
// chunk block to finish merges the C partials. Merging moves each floored partial to the row's
// larger base by an arithmetic right shift: floor(a 2^-s) <= a 2^-s < floor(a 2^-s) + lost, so
// the row's sums stay of the form [acc, acc + lost count] in units of the common base, the form
// the final rounding takes. With C = 1 the block finishes the row itself.
__global__ void __launch_bounds__(EA_T2_THREADS) ea_tier2(Params P) {
    __shared__ T2Smem S;
    __shared__ int s_last;
    const int tid = threadIdx.x;
    const int cnt = *P.wl_cnt;
    const int C = cnt >= (int)gridDim.x ? 1 : (int)gridDim.x / max(cnt, 1);
    const int64_t items = (int64_t)cnt * C;
    if ((int64_t)blockIdx.x >= items) return;  // no listed row for this block (the usual case)
    for (int i = tid; i < 256; i += EA_T2_THREADS) {
        S.T1[i] = u64_as_f64(EA_T1_BITS[i]);
        S.T2[i] = u64_as_f64(EA_T2_BITS[i]);
    }
    __syncthreads();
    const int d = P.g.head_dim, dv = P.g.head_dim_v;
    const int Hq = P.g.num_q_heads, T = P.g.num_tokens;
    int32_t* Mw = P.t2M + (int64_t)blockIdx.x * P.t2_keys;
    int64_t* Ew = P.t2E + (int64_t)blockIdx.x * P.t2_keys;
    T2Part* parts = (T2Part*)P.t2part;
    for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
        const int slot = (int)(item / C), chunk = (int)(item % C);
        const int64_t row = P.wl[slot];
        const int64_t b = row / ((int64_t)T * Hq);
        const int t = (int)((row / Hq) % T), hq = (int)(row % Hq);
        const int hk = hq / P.grp;
        const int64_t tok = b * T + t;
        // the row's visible keys (vis_prefix, vis_tree_bits: the set tier 1 attends); this block
        // takes keys [jc0, jc1) of them
        const int64_t slen = P.seq_len[b];
        const int64_t L = vis_prefix(P.kv_len[tok], slen);
        const uint64_t mask =
            P.tree_mask ? vis_tree_bits(P.tree_mask[tok], (int64_t)P.tree_base[b], L, slen) : 0ull;
        const int64_t nkeys = L + __popcll(mask);
        const int64_t csz = (nkeys + C - 1) / C;
        const int64_t jc0 = min(nkeys, (int64_t)chunk * csz), jc1 = min(nkeys, jc0 + csz);
        const int64_t nkc = jc1 - jc0;
        const int64_t obase = b * P.g.o_seq_stride + (int64_t)t * P.g.o_tok_stride + (int64_t)hq * P.g.o_head_stride;
        // the flag starts at 0 before any wave can raise it (a NaN/inf q element below)
        if (tid == 0) S.flag = 0;
        __syncthreads();
        const uint16_t* qr = P.q + b * P.g.q_seq_stride + (int64_t)t * P.g.q_tok_stride + (int64_t)hq * P.g.q_head_stride;
        for (int i = tid; i < d; i += EA_T2_THREADS) {
            uint32_t x = qr[i];
            int f = (x >> 7) & 0xFF;
            int m = (int)(x & 0x7F) | (f ? 0x80 : 0);
            S.qm[i] = (x & 0x8000) ? -m : m;
            S.qe[i] = (f ? f : 1) - 134;
            if (f == 0xFF) atomicMax(&S.flag, 2);
        }
        __syncthreads();
        int myflag = 0;
        if (nkeys > P.t2_keys) myflag = 1;  // workspace too small: not certified
        // ---- scores, logits, weights: one key per thread, its K row read coalesced in 16-dim
        // chunks twice (the lead exponent, then the window sum in 128 bits)
        const int wv = tid >> 6, ln = tid & 63;
        uint64_t tq0 = __builtin_amdgcn_s_memtime();
        // phase clocks (P.timers set): slots 9..13 = scores, Z, N maxima, N sums, rounding
        auto t2tick = [&](int ts) __attribute__((always_inline)) {
            if (P.timers) {
                const uint64_t tn = __builtin_amdgcn_s_memtime();
                if (tid == 0) atomicAdd((unsigned long long*)&P.timers[ts], (unsigned long long)(tn - tq0));
                tq0 = tn;
            }
        };
        const int64_t tb = P.tree_mask ? P.tree_base[b] : 0;
        auto key_n = [&](int64_t j) -> int64_t {
            if (j < L) return j;
            uint64_t m = mask;
            for (int64_t cc = j - L; cc > 0; --cc) m &= m - 1;
            return tb + (__ffsll((long long)m) - 1);
        };
        int64_t emax = INT64_MIN;
        // one key per thread, its K row in registers (16-byte loads when rows are aligned)
        const bool k16 = (((uintptr_t)P.k | (uintptr_t)(P.g.k_page_stride * 2) | (uintptr_t)(P.g.k_slot_stride * 2) |
                           (uintptr_t)(P.g.k_head_stride * 2)) & 15) == 0 && d == 128;
        for (int64_t jr = tid; jr < nkc && !myflag && S.flag < 2; jr += EA_T2_THREADS) {
            const uint16_t* kr = P.k + kv_off(P, b, key_n(jc0 + jr), hk, 0);
            // 16 dims (8 dwords) at a time, read twice: the lead exponent, then the window sum
            auto kchunk = [&](int c16, uint32_t (&kw)[8]) __attribute__((always_inline)) {
                if (k16) {
                    const uint4 u0 = ((const uint4*)kr)[2 * c16], u1 = ((const uint4*)kr)[2 * c16 + 1];
                    kw[0] = u0.x; kw[1] = u0.y; kw[2] = u0.z; kw[3] = u0.w;
                    kw[4] = u1.x; kw[5] = u1.y; kw[6] = u1.z; kw[7] = u1.w;
                } else {
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        const int i = 16 * c16 + 2 * c;
                        kw[c] = (i < d ? (uint32_t)kr[i] : 0u) | ((i + 1 < d ? (uint32_t)kr[i + 1] : 0u) << 16);
                    }
                }
            };
            int lmax = INT_MIN;
            bool bad = false;
            for (int c16 = 0; c16 < EA_MAXD / 16; ++c16) {
                uint32_t kw[8];
                kchunk(c16, kw);
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int i = 16 * c16 + e;
                    const uint32_t x = (kw[e >> 1] >> (16 * (e & 1))) & 0xFFFF;
                    const int f = (x >> 7) & 0xFF;
                    bad |= f == 0xFF;
                    const int m = (int)(x & 0x7F) | (f ? 0x80 : 0);
                    const int pr = S.qm[i] * ((x & 0x8000) ? -m : m);
                    if (pr) lmax = max(lmax, S.qe[i] + (f ? f : 1) - 134 + (31 - __clz(pr < 0 ? -pr : pr)));
                }
            }
            if (bad) {
                atomicMax(&S.flag, 2);
                break;
            }
            int32_t M = 1 << 23;
            int64_t E = -23;
            if (lmax != INT_MIN && P.am != 0) {
                const int base = lmax + 1 - 120;
                i128 acc = 0;
                uint64_t err = 0;
                for (int c16 = 0; c16 < EA_MAXD / 16; ++c16) {
                    uint32_t kw[8];
                    kchunk(c16, kw);
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int i = 16 * c16 + e;
                        const uint32_t x = (kw[e >> 1] >> (16 * (e & 1))) & 0xFFFF;
                        const int f = (x >> 7) & 0xFF;
                        const int m = (int)(x & 0x7F) | (f ? 0x80 : 0);
                        const int pr = S.qm[i] * ((x & 0x8000) ? -m : m);
                        if (!pr) continue;
                        int lost;
                        acc += floor_shift128((i128)pr, (int64_t)S.qe[i] + (f ? f : 1) - 134 - base, &lost);
                        err += (uint64_t)lost;
                    }
                }
                uint32_t tlo = 0, thi = 0;
                const int slo = rn32_prod(P.am, acc, P.ae + base, &tlo);
                const int shi = err ? rn32_prod(P.am, acc + (i128)err, P.ae + base, &thi) : slo;
                if (!err) thi = tlo;
                if (slo == 2 && shi == 2) {
                    atomicMax(&S.flag, 2);  // |alpha s| rounds above fp32 max: domain error
                    break;
                }
                if (slo != 0 || shi != 0 || tlo != thi) {
                    myflag = 1;
                    break;
                }
                int32_t Mi;
                int32_t Ei;
                if (weight_f64(tlo, S.T1, S.T2, &Mi, &Ei) == 0) {
                    M = Mi;
                    E = Ei;
                } else if (weight_wide(tlo, &M, &E)) {
                    myflag = 1;
                    break;
                }
            }
            Mw[jr] = M;
            Ew[jr] = E;
            emax = max(emax, E + 23);
        }
        if (myflag) atomicMax(&S.flag, 1);
        __syncthreads();
        int64_t R;
        block_max_i64(S, emax, &R);
        t2tick(9);
        int fl = S.flag;
        // F: every chunk sums against windows of the row's key count, so the partials merge
        int key_log2 = 0;
        while (((int64_t)1 << key_log2) < nkeys) ++key_log2;
        const int F = 126 - key_log2;
        i128 z = 0;
        uint64_t ze = 0;
        if (fl == 0 && nkc > 0) {
            // Z
            for (int64_t jr = tid; jr < nkc; jr += EA_T2_THREADS) {
                int lost;
                z += floor_shift128((i128)Mw[jr], Ew[jr] - (R - F), &lost);
                ze += (uint64_t)lost;
            }
            block_reduce_i128(S, &z, &ze);
            t2tick(10);
            // N per channel, key-parallel: wave wv takes keys wv, wv + 8, ... of the chunk; lane
            // ln channels 2 ln and 2 ln + 1. Pass 1: NR_c = max_j (E_j + 24 + lead(v_jc)); pass
            // 2: the 128-bit sums of floor(M_j v_jc 2^(E_j + e_jc - base_c)) and their lost
            // counts, base_c = NR_c - F; partials reduced over the waves through LDS.
            // batches of 16 keys per wave: lane ln finds key jb + ln's V row, the row offsets are
            // broadcast and the batch's V elements loaded together (independent loads in flight)
            uint32_t vx[16][2];
            auto load_batch = [&](int64_t jb, int nk) __attribute__((always_inline)) {
                const int64_t myoff = ln < nk ? kv_off(P, b, key_n(jc0 + jb + ln), hk, 1) : 0;
#pragma unroll
                for (int kk = 0; kk < 16; ++kk) {
                    const int64_t o = __shfl(myoff, kk, 64);
#pragma unroll
                    for (int h = 0; h < 2; ++h) vx[kk][h] = (kk < nk && 2 * ln + h < dv) ? (uint32_t)P.v[o + 2 * ln + h] : 0u;
                }
            };
            const int64_t nvb = (nkc + 16 * EA_T2_WAVES - 1) / (16 * EA_T2_WAVES);
            int64_t nr[2] = {INT64_MIN, INT64_MIN};
            bool vbad = false;
            for (int64_t bt = 0; bt < nvb; ++bt) {
                const int64_t jb = (bt * EA_T2_WAVES + wv) * 16;
                if (jb >= nkc) break;
                const int nk = (int)min((int64_t)16, nkc - jb);
                load_batch(jb, nk);
#pragma unroll
                for (int kk = 0; kk < 16; ++kk) {
                    if (kk >= nk) continue;
                    const int64_t e = Ew[jb + kk] + 24;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                    const uint32_t x = vx[kk][h];
                    if (!(x & 0x7FFF)) continue;
                    const int f = (x >> 7) & 0xFF;
                    if (f == 0xFF) vbad = true;
                    const int m = (int)(x & 0x7F) | (f ? 0x80 : 0);
                    nr[h] = max(nr[h], e + (f ? f : 1) - 134 + (31 - __clz(m)));
                    }
                }
            }
            if (vbad) atomicMax(&S.flag, 2);  // NaN/inf in a visible V row: a domain error
            t2tick(11);
#pragma unroll
            for (int h = 0; h < 2; ++h)
                if (2 * ln + h < EA_MAXDV) S.nrw[wv][2 * ln + h] = nr[h];
            __syncthreads();
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int c = 2 * ln + h;
                nr[h] = INT64_MIN;
                for (int q = 0; q < EA_T2_WAVES; ++q) nr[h] = max(nr[h], S.nrw[q][c]);
            }
            i128 acc[2] = {0, 0};
            uint64_t err[2] = {0, 0};
            for (int64_t bt = 0; bt < nvb; ++bt) {
                const int64_t jb = (bt * EA_T2_WAVES + wv) * 16;
                if (jb >= nkc) break;
                const int nk = (int)min((int64_t)16, nkc - jb);
                load_batch(jb, nk);
#pragma unroll
                for (int kk = 0; kk < 16; ++kk) {
                    if (kk >= nk) continue;
                    const int64_t Ej = Ew[jb + kk];
                    const int64_t Mj = Mw[jb + kk];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint32_t x = vx[kk][h];
                        if (!(x & 0x7FFF) || nr[h] == INT64_MIN) continue;
                        const int f = (x >> 7) & 0xFF;
                        const int m = (int)(x & 0x7F) | (f ? 0x80 : 0);
                        const int64_t vm = (x & 0x8000) ? -m : m;
                        int lost;
                        acc[h] += floor_shift128((i128)(Mj * vm), Ej + (f ? f : 1) - 134 - (nr[h] - F), &lost);
                        err[h] += (uint64_t)lost;
                    }
                }
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int c = 2 * ln + h;
                if (c < EA_MAXDV) {
                    S.ahi[wv][c] = (uint64_t)((u128)acc[h] >> 64);
                    S.alo[wv][c] = (uint64_t)(u128)acc[h];
                    S.aer[wv][c] = err[h];
                }
            }
            __syncthreads();
            t2tick(12);
            fl = S.flag;
        }
        // the chunk's channel sums (over the waves: one base per channel, exact 128-bit adds)
        auto channel_sum = [&](int c, int64_t* NR, i128* acc, uint64_t* err) __attribute__((always_inline)) {
            *NR = INT64_MIN;
            u128 accu = 0;
            uint64_t e = 0;
            for (int q = 0; q < EA_T2_WAVES; ++q) {
                *NR = max(*NR, S.nrw[q][c]);
                accu += ((u128)S.ahi[q][c] << 64) | S.alo[q][c];
                e += S.aer[q][c];
            }
            *acc = (i128)accu;
            *err = e;
        };
        // certified RN(N_c / Z) into the output, N_c in [acc, acc + err] 2^(NR - F), Z in
        // [zz, zz + zze] 2^(RR - F); false when the interval straddles a rounding boundary
        auto round_out = [&](int c, int64_t NR, i128 acc, uint64_t err, i128 zz, uint64_t zze, int64_t RR) {
            uint32_t bits = 0;
            bool ok = true;
            if (NR != INT64_MIN)
                ok = certify_quotient(acc, acc + (i128)err, zz, zz + (i128)zze, NR - RR, P.out_fp32, &bits);
            if (P.out_fp32) ((uint32_t*)P.out)[obase + c] = bits;
            else ((uint16_t*)P.out)[obase + c] = (uint16_t)bits;
            return ok;
        };
        // flags, zero output for a flagged row, stats: once per row
        auto finish_row = [&](int f) __attribute__((always_inline)) {
            if (f != 0) {
                for (int c = tid; c < dv; c += EA_T2_THREADS) {
                    if (P.out_fp32) ((uint32_t*)P.out)[obase + c] = 0;
                    else ((uint16_t*)P.out)[obase + c] = 0;
                }
            }
            if (tid == 0) {
                P.flags[row] = (uint8_t)f;
                if (P.stats) {
                    if (f == 0) atomicAdd((unsigned long long*)&P.stats[2], 1ull);
                    if (f == 1) atomicAdd((unsigned long long*)&P.stats[3], 1ull);
                    if (f == 2) atomicAdd((unsigned long long*)&P.stats[4], 1ull);
                }
            }
        };
        if (C == 1) {
            if (fl == 0 && nkeys > 0) {
                bool ok = true;
                for (int c = tid; c < dv; c += EA_T2_THREADS) {
                    int64_t NR;
                    i128 acc;
                    uint64_t err;
                    channel_sum(c, &NR, &acc, &err);
                    if (!round_out(c, NR, acc, err, z, ze, R)) ok = false;
                }
                if (!ok) atomicMax(&S.flag, 1);
                __syncthreads();
                t2tick(13);
                fl = S.flag;
            } else if (fl == 0) {
                for (int c = tid; c < dv; c += EA_T2_THREADS) {
                    if (P.out_fp32) ((uint32_t*)P.out)[obase + c] = 0;
                    else ((uint16_t*)P.out)[obase + c] = 0;
                }
            }
            finish_row(fl);
            __syncthreads();
            continue;
        }
        // ---- C > 1: this chunk's partial (item < gridDim.x slots), then the row's last chunk
        // block merges. Release: every thread's partial stores are visible at device scope (other
        // XCDs included) before the count moves; acquire: the merging block reads the others'
        // partials only after it has seen the full count.
        T2Part& pt = parts[item];
        const bool have = fl == 0 && nkc > 0;
        if (tid == 0) {
            pt.R = have ? R : INT64_MIN;
            pt.flag = fl;
            pt.zhi = have ? (uint64_t)((u128)z >> 64) : 0;
            pt.zlo = have ? (uint64_t)(u128)z : 0;
            pt.ze = have ? ze : 0;
        }
        for (int c = tid; c < dv; c += EA_T2_THREADS) {
            int64_t NR = INT64_MIN;
            i128 acc = 0;
            uint64_t err = 0;
            if (have) channel_sum(c, &NR, &acc, &err);
            pt.nr[c] = NR;
            pt.nhi[c] = (uint64_t)((u128)acc >> 64);
            pt.nlo[c] = (uint64_t)(u128)acc;
            pt.ner[c] = err;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __syncthreads();
        if (tid == 0) s_last = atomicAdd(&P.wl_cnt[1 + slot], 1) == C - 1;
        __syncthreads();
        if (s_last) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            const T2Part* rp = parts + (int64_t)slot * C;
            int rf = 0;
            int64_t RR = INT64_MIN;
            for (int k = 0; k < C; ++k) {
                rf = max(rf, rp[k].flag);
                RR = max(RR, rp[k].R);
            }
            if (rf == 0 && RR != INT64_MIN) {
                // Z over the chunks, each moved to base RR - F (thread k takes chunk k)
                i128 zz = 0;
                uint64_t zze = 0;
                for (int k = tid; k < C; k += EA_T2_THREADS) {
                    if (rp[k].R == INT64_MIN) continue;
                    const i128 zb = (i128)(((u128)rp[k].zhi << 64) | rp[k].zlo);
                    int lost;
                    zz += floor_shift128(zb, rp[k].R - RR, &lost);
                    zze += rp[k].ze + (uint64_t)lost;
                }
                block_reduce_i128(S, &zz, &zze);
                bool ok = true;
                for (int c = tid; c < dv; c += EA_T2_THREADS) {
                    int64_t NR = INT64_MIN;
                    for (int k = 0; k < C; ++k) NR = max(NR, rp[k].nr[c]);
                    i128 acc = 0;
                    uint64_t err = 0;
                    if (NR != INT64_MIN)
                        for (int k = 0; k < C; ++k) {
                            if (rp[k].nr[c] == INT64_MIN) continue;
                            const i128 nb = (i128)(((u128)rp[k].nhi[c] << 64) | rp[k].nlo[c]);
                            int lost;
                            acc += floor_shift128(nb, rp[k].nr[c] - NR, &lost);
                            err += rp[k].ner[c] + (uint64_t)lost;
                        }
                    if (!round_out(c, NR, acc, err, zz, zze, RR)) ok = false;
                }
                if (tid == 0) S.flag = 0;
                __syncthreads();
                if (!ok) atomicMax(&S.flag, 1);
                __syncthreads();
                rf = S.flag;
            } else if (rf == 0) {
                for (int c = tid; c < dv; c += EA_T2_THREADS) {
                    if (P.out_fp32) ((uint32_t*)P.out)[obase + c] = 0;
                    else ((uint16_t*)P.out)[obase + c] = 0;
                }
            }
            finish_row(rf);
            if (tid == 0) P.wl_cnt[1 + slot] = 0;  // the row's count, ready for the next launch
        }
        __syncthreads();
    }
}

// Lists every row for tier 2 (ea_options.force_tier2); runs after tier 1, so nothing else appends.
__global__ void __launch_bounds__(256) ea_list_all(Params P) {
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r < P.rows) P.wl[r] = (int32_t)r;
    if (r == 0) *P.wl_cnt = (int32_t)P.rows;
}

// The host exact tier's input for one row: its q row, then the K rows and the V rows of its
// visible keys (the prefix, then the tree keys in bit order: vis_prefix, vis_tree_bits), packed in
// dst as [q d][K nkeys x d][V nkeys x dv], one element per thread.
__global__ void __launch_bounds__(256) ea_gather_row(Params P, int64_t row, int64_t nkeys, uint16_t* dst) {
    const int d = P.g.head_dim, dv = P.g.head_dim_v, T = P.g.num_tokens, Hq = P.g.num_q_heads;
    const int64_t b = row / ((int64_t)T * Hq);
    const int t = (int)((row / Hq) % T), hq = (int)(row % Hq);
    const int hk = hq / P.grp;
    const int64_t tok = b * T + t;
    const int64_t slen = P.seq_len[b];
    const int64_t L = vis_prefix(P.kv_len[tok], slen);
    const int64_t tb = P.tree_mask ? P.tree_base[b] : 0;
    const uint64_t mask = P.tree_mask ? vis_tree_bits(P.tree_mask[tok], tb, L, slen) : 0ull;
    const int64_t total = d + nkeys * (int64_t)(d + dv);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        if (i < d) {
            dst[i] = P.q[b * P.g.q_seq_stride + (int64_t)t * P.g.q_tok_stride + (int64_t)hq * P.g.q_head_stride + i];
            continue;
        }
        int64_t r = i - d;
        const int isv = r >= nkeys * d ? 1 : 0;
        if (isv) r -= nkeys * d;
        const int wdt = isv ? dv : d;
        const int64_t j = r / wdt;
        const int e = (int)(r % wdt);
        int64_t n = j;
        if (j >= L) {
            uint64_t m = mask;
            for (int64_t c = j - L; c > 0; --c) m &= m - 1;
            n = tb + (__ffsll((long long)m) - 1);
        }
        dst[i] = (isv ? P.v : P.k)[kv_off(P, b, n, hk, isv) + e];
    }
}

// ------------------------------------------------------------------------------------------------
// KV append: new key rows scattered into the paged pools and block-table entries written, in one
// launch (grid-stride, U = 16-byte chunks when every row is 16-byte aligned, else uint16).
// Destinations outside the pool or the table are skipped.
// ------------------------------------------------------------------------------------------------
template <typename U>
__global__ void __launch_bounds__(256) ea_kv_append(U* kp, U* vp, int64_t pool_rows, int64_t row_u, const U* kn,
                                                    const U* vn, const int64_t* dst, int64_t n, int32_t* bt,
                                                    int64_t bt_entries, const int64_t* bt_pos, const int32_t* bt_val,
                                                    int64_t nbt) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t x0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (int64_t x = x0; x < n * row_u; x += stride) {
        const int64_t i = x / row_u, c = x - i * row_u;
        const int64_t d = dst[i];
        if (d < 0 || d >= pool_rows) continue;
        kp[d * row_u + c] = kn[x];
        vp[d * row_u + c] = vn[x];
    }
    for (int64_t j = x0; j < nbt; j += stride) {
        const int64_t pos = bt_pos[j];
        if (pos >= 0 && pos < bt_entries) bt[pos] = bt_val[j];
    }
}

// ------------------------------------------------------------------------------------------------
// Known-answer kernels over the device helpers
// ------------------------------------------------------------------------------------------------
__global__ void ea_kat_weight(int64_t n, const uint32_t* t, int32_t* M, int64_t* E, int32_t* st, int32_t* M2,
                              int64_t* E2, int32_t* st2) {
    __shared__ double T1[256], T2[256];
    for (int i = threadIdx.x; i < 256; i += blockDim.x) {
        T1[i] = u64_as_f64(EA_T1_BITS[i]);
        T2[i] = u64_as_f64(EA_T2_BITS[i]);
    }
    __syncthreads();
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int32_t m = 0, e = 0;
    st[i] = weight_f64(t[i], T1, T2, &m, &e);
    M[i] = m;
    E[i] = e;
    int32_t m2 = 0;
    int64_t e2 = 0;
    st2[i] = weight_wide(t[i], &m2, &e2);
    M2[i] = m2;
    E2[i] = e2;
}

__global__ void __launch_bounds__(64) ea_kat_wave_max(int64_t nwaves, const int32_t* in, int32_t* out) {
    if (blockIdx.x >= nwaves) return;
    int v = wave_max_dpp(in[blockIdx.x * 64 + threadIdx.x]);
    out[blockIdx.x * 64 + threadIdx.x] = v;
}

__global__ void ea_kat_round(int64_t n, const double* x, const double* r, int32_t fp32, uint32_t* bits, int32_t* ok) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t bb = 0;
    ok[i] = certify_round(x[i], r[i], fp32, &bb) ? 1 : 0;
    bits[i] = bb;
}

__global__ void ea_kat_rn32_prod(int64_t n, const int32_t* am, const int64_t* x_hi, const uint64_t* x_lo,
                                 const int32_t* E, uint32_t* bits, int32_t* status) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const i128 X = (i128)(((u128)(uint64_t)x_hi[i] << 64) | x_lo[i]);
    uint32_t bb = 0;
    status[i] = rn32_prod(am[i], X, E[i], &bb);
    bits[i] = bb;
}

__global__ void ea_kat_round_ratio(int64_t n, const uint64_t* ah, const uint64_t* al, const uint64_t* bh,
                                   const uint64_t* bl, const int32_t* E, const int32_t* neg, int32_t fp32, uint32_t* bits,
                                   int32_t* ov) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const u128 a = ((u128)ah[i] << 64) | al[i], b = ((u128)bh[i] << 64) | bl[i];
    quant y;
    const int st = rn_quotient(a, b, E[i], fp32 ? 24 : 8, fp32 ? -149 : -133, &y);
    ov[i] = st;
    bits[i] = st ? 0u : fmt_bits(y.Q, y.qe, neg[i] != 0, fp32);
}

// v: per case Nlo, Nhi, Zlo, Zhi as (hi, lo) word pairs, then sh (9 int64)
__global__ void ea_kat_certify_quotient(int64_t n, const int64_t* v, int32_t fp32, uint32_t* bits, int32_t* ok) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t* c = v + 9 * i;
    auto s128 = [](int64_t hi, int64_t lo) { return (i128)(((u128)(uint64_t)hi << 64) | (uint64_t)lo); };
    uint32_t b = 0;
    ok[i] = certify_quotient(s128(c[0], c[1]), s128(c[2], c[3]), s128(c[4], c[5]), s128(c[6], c[7]), c[8], fp32, &b)
                ? 1
                : 0;
    bits[i] = b;
}

// ------------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------------
namespace {

struct Plan {
    int nsplit, split_len, rb, nrb, r_seg, grp, nseg, pshift, dlog;
    int64_t rows;
    size_t off_q64, off_qinfo, off_qn, off_pR, off_pn, off_pZ, off_pN, off_pV, off_wl, off_cnt, off_t2M, off_t2E, total;
    size_t off_pfq, off_pfqm, off_pfkv, off_pfscr, off_pfpart, off_dq, off_t2part;
    int t2_keys;
    int prefill, pf_ntiles, pf_nrb, pf_nsplit, pf_tps;
    // the decode kernel's equal-share decomposition (Params::dq_*): dq = 1 when the geometry may
    // take it (the pointer checks come at launch); nsplit_gen = the general kernel's uniform split
    // count, nsplit = nsplit_gen + 1 partial slots per unit for the decode kernel's pieces
    int dq, nsplit_gen, dq_units, dq_min_share, dq_max_tiles, dq_rec_off;
};

// most blocks the decode kernel's equal-share decomposition launches (the plan array's size)
#define EA_DQ_MAX_BLOCKS 4096

size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

int make_plan(const ea_geometry* g, const ea_options* o, Plan* pl) {
    if (!g || !o) return -1;
    if (g->num_seqs < 0 || g->num_tokens <= 0 || g->num_q_heads <= 0 || g->num_kv_heads <= 0) return -1;
    if (g->num_q_heads % g->num_kv_heads) return -1;
    if (g->head_dim <= 0 || g->head_dim > EA_MAXD || (g->head_dim & 7)) return -1;
    if (g->head_dim_v <= 0 || g->head_dim_v > EA_MAXDV || (g->head_dim_v & 1)) return -1;
    if (g->page_size <= 0 || (g->page_size & (g->page_size - 1))) return -1;
    if (g->max_seq_len < 0) return -1;
    if (o->splits < 0) return -2;
    if (o->kernel < EA_KERNEL_AUTO || o->kernel > EA_KERNEL_GENERAL) return -2;
    if (o->prefill_waves != 0 && o->prefill_waves != 4 && o->prefill_waves != 8) return -2;
    pl->grp = g->num_q_heads / g->num_kv_heads;
    pl->r_seg = g->num_tokens * pl->grp;
    // rows per block: the d = 128 decode kernel takes 1- or 2-row blocks (two waves per SIMD; a
    // 4-row block needs more than 256 VGPRs, runs at one wave per SIMD and measured 4-14% slower
    // on every multi-row shape: GQA 4 and 8 decode, 4-16 query tokens), the general split kernel
    // 1, 2 or 4
    const bool dec_rows = g->head_dim == 128 && g->head_dim_v == 128 && o->kernel != EA_KERNEL_GENERAL && !o->timers;
    pl->rb = dec_rows ? std::min(pl->r_seg, 2) : (pl->r_seg >= 3 ? 4 : pl->r_seg);
    pl->nrb = (pl->r_seg + pl->rb - 1) / pl->rb;
    pl->nseg = g->num_seqs * g->num_kv_heads;
    pl->rows = (int64_t)g->num_seqs * g->num_tokens * g->num_q_heads;
    int ps = 0;
    while ((1 << ps) < g->page_size) ++ps;
    pl->pshift = ps;
    int dl = 0;
    while ((1 << dl) < g->head_dim) ++dl;
    pl->dlog = dl;
    int maxlen = g->max_seq_len > 0 ? g->max_seq_len : 1;
    int ns = o->splits;
    if (ns == 0) {
        // enough work items for 256 CUs x 2 blocks, splits of at least 256 keys
        int64_t items = (int64_t)pl->nseg * pl->nrb;
        ns = 1;
        while (items * ns < 1024 && (int64_t)maxlen / (ns * 2) >= 256) ns *= 2;
        // and splits of at most 2048 keys: with sequence lengths that differ (only their maximum
        // is known here), long splits leave the blocks of short sequences idle while the longest
        // block runs, and the last round of blocks is sparse (C5, 8K-131K keys: 8 splits 1.36 ms,
        // 32 splits 1.19-1.21 ms, 63 splits 1.16-1.19 ms per step)
        while ((int64_t)maxlen / ns > 2048 && ns < 1024) ns *= 2;
    }
    int sl = (maxlen + ns - 1) / ns;
    sl = (sl + EA_TILE - 1) / EA_TILE * EA_TILE;
    if (sl < EA_TILE) sl = EA_TILE;
    pl->split_len = sl;
    pl->nsplit = (maxlen + sl - 1) / sl;
    if (pl->nsplit < 1) pl->nsplit = 1;
    pl->nsplit_gen = pl->nsplit;
    // the d = 128 decode kernel may run this step (ea_launch_decode also checks the pointers):
    // its pieces need nsplit + 1 partial slots per unit
    const int64_t max_tiles = ((int64_t)maxlen + 63) / 64;
    int pf_nt = 0, pf_nr = 0;
    pl->dq = g->head_dim == 128 && g->head_dim_v == 128 && o->kernel != EA_KERNEL_GENERAL && !o->timers &&
             !ea_prefill_eligible(*g, pl->grp, o->kernel, &pf_nt, &pf_nr) && pl->rows < ((int64_t)1 << 30) &&
             (int64_t)maxlen + 64 < ((int64_t)1 << 30) &&
             (int64_t)pl->nseg * pl->nrb * max_tiles < ((int64_t)1 << 30) &&
             (int64_t)pl->nseg * pl->nrb < ((int64_t)1 << 24);
    pl->dq_units = pl->nseg * pl->nrb;
    pl->dq_max_tiles = (int)max_tiles;
    pl->dq_min_share = (int)((max_tiles + pl->nsplit_gen - 1) / pl->nsplit_gen);
    if (pl->dq) pl->nsplit = pl->nsplit_gen + 1;
    int64_t R = pl->rows;
    int dv = g->head_dim_v;
    size_t off = 0;
    pl->off_q64 = off; off = align_up(off + (size_t)R * EA_MAXD * 8);
    pl->off_qinfo = off; off = align_up(off + (size_t)R * 5 * 4);
    pl->off_qn = off; off = align_up(off + (size_t)R * 4 * 8);
    pl->off_pR = off; off = align_up(off + (size_t)pl->nsplit * R * 4);
    pl->off_pn = off; off = align_up(off + (size_t)pl->nsplit * R * 4);
    pl->off_pZ = off; off = align_up(off + (size_t)pl->nsplit * R * 8);
    pl->off_pN = off; off = align_up(off + (size_t)pl->nsplit * R * dv * 8);
    pl->off_pV = off; off = align_up(off + (size_t)pl->nsplit * pl->nseg * pl->nrb * dv * 4);
    pl->off_wl = off; off = align_up(off + (size_t)(R > 0 ? R : 1) * 4);
    pl->off_cnt = off; off = align_up(off + 4 * (1 + EA_T2_BLOCKS));
    pl->off_t2part = off; off = align_up(off + EA_T2_BLOCKS * sizeof(T2Part));
    pl->off_dq = off;
    pl->dq_rec_off = (3 + pl->dq_units + 3) & ~3;  // 16-byte aligned block records after S
    if (pl->dq) off = align_up(off + (size_t)(pl->dq_rec_off + 4 * EA_DQ_MAX_BLOCKS) * 4);
    pl->t2_keys = maxlen + 64;
    pl->off_t2M = off; off = align_up(off + (size_t)EA_T2_BLOCKS * pl->t2_keys * 4);
    pl->off_t2E = off; off = align_up(off + (size_t)EA_T2_BLOCKS * pl->t2_keys * 8);
    pl->prefill = ea_prefill_eligible(*g, pl->grp, o->kernel, &pl->pf_ntiles, &pl->pf_nrb) ? 1 : 0;
    pl->off_pfq = pl->off_pfqm = pl->off_pfkv = pl->off_pfscr = pl->off_pfpart = 0;
    pl->pf_nsplit = pl->pf_tps = 1;
    if (pl->prefill) {
        pl->off_pfq = off; off = align_up(off + (size_t)R * 512);
        pl->off_pfqm = off; off = align_up(off + (size_t)R * sizeof(PfQMeta));
        if (o->kv_digits) {
            // the caller's digit cache holds the K/V tiles: nothing to slice into the workspace
            if (o->kv_digits_tiles < pl->pf_ntiles) return -1;
        } else {
            pl->off_pfkv = off; off = align_up(off + (size_t)pl->nseg * pl->pf_ntiles * EA_PF_TILE_BYTES);
        }
        // key splits when the (segment, row block) grid alone leaves CUs idle (one prefill block
        // fills a CU's LDS): double the splits while the grid is under 256 blocks and every split
        // keeps at least 16 tiles; a caller's split count is taken as given
        int ns = 1;
        if (o->splits > 0) {
            ns = o->splits;
        } else {
            while ((int64_t)pl->nseg * pl->pf_nrb * ns < 256 && pl->pf_ntiles / (2 * ns) >= 16) ns *= 2;
        }
        pl->pf_tps = (pl->pf_ntiles + ns - 1) / ns;
        if (pl->pf_tps < 1) pl->pf_tps = 1;
        pl->pf_nsplit = (pl->pf_ntiles + pl->pf_tps - 1) / pl->pf_tps;
        if (pl->pf_nsplit < 1) pl->pf_nsplit = 1;
        pl->off_pfscr = off;
        off = align_up(off + (size_t)pl->nseg * pl->pf_nrb * pl->pf_nsplit * 512 * 32 * 8);
        pl->off_pfpart = off;
        if (pl->pf_nsplit > 1)
            off = align_up(off + (size_t)pl->pf_nsplit * R * (sizeof(PfPart) + 128 * 16));
        pl->nsplit = pl->pf_nsplit;  // the split count this step uses
    }
    pl->total = off;
    return 0;
}

int herr(hipError_t e) { return e == hipSuccess ? 0 : -100 - (int)e; }

}  // namespace

// The allocation-free entry point's workspace (ea_hip_attention_noalloc): one array per device,
// held by the device until the process ends. Host code never passes this name to a kernel or a
// copy (on the host it only stands for the symbol): it uses the device address that
// hipGetSymbolAddress returned for the current device, kept in scratch_ptr.
static __device__ __align__(256) unsigned char scratch[EA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int EA_MAX_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_ptr[EA_MAX_DEVICES] = {};

// The device address of `scratch` on the current device, looked up once per device (with that
// device current) and cached; 0 or -100 - e.
int scratch_address(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return herr(e);
    if (dev < 0 || dev >= EA_MAX_DEVICES) return -1;
    std::lock_guard<std::mutex> lk(scratch_mu);
    if (!scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return herr(e);
        if (!p) return -1;
        scratch_ptr[dev] = p;
    }
    *out = scratch_ptr[dev];
    return 0;
}

// ea_options.force_tier2: every row onto the tier-2 work list (after tier 1)
int list_all(const Params& P, const ea_options* o, unsigned blocks, hipStream_t st) {
    if (!o->force_tier2) return 0;
    hipLaunchKernelGGL(ea_list_all, dim3(blocks), dim3(256), 0, st, P);
    return herr(hipGetLastError());
}

}  // namespace

extern "C" {

const char* ea_hip_version(void) { return "exactattn_hip 0.1 (gfx950, fp64 tier 1, 128-bit tier 2)"; }

int ea_hip_workspace_size(const ea_geometry* g, const ea_options* o, size_t* bytes, int32_t* nsplit) {
    Plan pl;
    int rc = make_plan(g, o, &pl);
    if (rc) return rc;
    if (bytes) *bytes = pl.total;
    if (nsplit) *nsplit = pl.prefill ? pl.nsplit : pl.nsplit_gen;  // the decode kernel adds one partial slot
    return 0;
}

int ea_hip_reads_kv_digits(const ea_geometry* g, const ea_options* o, int32_t* reads) {
    Plan pl;
    int rc = make_plan(g, o, &pl);
    if (rc) return rc;
    if (reads) *reads = (pl.prefill && o->kv_digits) ? 1 : 0;  // the test ea_hip_attention makes
    return 0;
}

int ea_hip_attention(const ea_geometry* g, const ea_buffers* bf, const ea_options* o, void* workspace,
                     size_t workspace_bytes, ea_stream_t stream) {
    Plan pl;
    int rc = make_plan(g, o, &pl);
    if (rc) return rc;
    uint32_t ab = o->alpha_bits;
    // an empty batch reads and writes nothing: no buffer or workspace is needed for it
    if (pl.rows == 0) return ((ab >> 23) & 0xFF) == 0xFF ? -3 : 0;
    if (!bf || !bf->q || !bf->k || !bf->v || !bf->seq_len || !bf->kv_len || !bf->out || !bf->flags) return -1;
    if (bf->tree_mask && !bf->tree_base) return -1;
    if (workspace_bytes < pl.total || (!workspace && pl.total)) return -2;
    if (((ab >> 23) & 0xFF) == 0xFF) return -3;
    Params P;
    memset(&P, 0, sizeof(P));
    P.g = *g;
    P.q = bf->q; P.k = bf->k; P.v = bf->v;
    P.seq_len = bf->seq_len; P.kv_len = bf->kv_len; P.bt = bf->block_table; P.bt_off = bf->block_table_offset;
    P.tree_mask = bf->tree_mask; P.tree_base = bf->tree_base;
    P.out = bf->out; P.flags = bf->flags; P.stats = o->stats; P.merge_order = o->merge_order;
    P.timers = o->timers;
    float af;
    memcpy(&af, &ab, 4);
    P.alpha = (double)af;
    {
        int ex = (ab >> 23) & 0xFF;
        int32_t fr = ab & 0x7FFFFF;
        int32_t m = ex ? (fr | 0x800000) : fr;
        P.am = (ab >> 31) ? -m : m;
        P.ae = ex ? ex - 150 : -149;
    }
    P.out_fp32 = o->out_fp32 ? 1 : 0;
    P.nsplit = pl.nsplit; P.split_len = pl.split_len;
    P.grp = pl.grp; P.r_seg = pl.r_seg; P.rb = pl.rb; P.nrb = pl.nrb; P.nseg = pl.nseg;
    P.pshift = pl.pshift; P.dlog = pl.dlog; P.rows = pl.rows;
    char* ws = (char*)workspace;
    P.q64 = (double*)(ws + pl.off_q64);
    P.qinfo = (int32_t*)(ws + pl.off_qinfo);
    P.qn = (double*)(ws + pl.off_qn);
    P.pR = (int32_t*)(ws + pl.off_pR);
    P.pn = (int32_t*)(ws + pl.off_pn);
    P.pZ = (double*)(ws + pl.off_pZ);
    P.pN = (double*)(ws + pl.off_pN);
    P.pV = (float*)(ws + pl.off_pV);
    P.wl = (int32_t*)(ws + pl.off_wl);
    P.wl_cnt = (int32_t*)(ws + pl.off_cnt);
    P.t2part = (void*)(ws + pl.off_t2part);
    P.t2M = (int32_t*)(ws + pl.off_t2M);
    P.t2E = (int64_t*)(ws + pl.off_t2E);
    P.t2_keys = pl.t2_keys;
    P.pfq = (uint8_t*)(ws + pl.off_pfq);
    P.pfqm = (void*)(ws + pl.off_pfqm);
    P.pfkv = (uint8_t*)(ws + pl.off_pfkv);
    if (pl.prefill && o->kv_digits) {
        P.pfkv = (uint8_t*)o->kv_digits;
        P.pf_kv_cached = 1;
        P.pf_kv_slot = o->kv_digits_slot;
    }
    P.pfscr = (double*)(ws + pl.off_pfscr);
    P.pf_ntiles = (pl.prefill && o->kv_digits) ? o->kv_digits_tiles : pl.pf_ntiles;
    P.pf_nrb = pl.pf_nrb;
    P.pf_waves = o->prefill_waves == 4 ? 4 : 8;
    P.pf_nsplit = pl.pf_nsplit;
    P.pf_tps = pl.pf_tps;
    P.pf_part = (void*)(ws + pl.off_pfpart);
    hipStream_t st = (hipStream_t)stream;
    unsigned rb4 = (unsigned)((pl.rows + 3) / 4);
    // the decode kernel with its equal-share plan, or the general kernel with uniform splits
    P.dq_stream = 0;
    bool use_decode = false;
    if (!pl.prefill) {
        P.nsplit = pl.nsplit_gen;
        use_decode = pl.dq && pl.nseg > 0 && ea_decode_eligible(P);
        int slots = 0, cus = 0;
        if (use_decode && (rc = ea_decode_slots(P, &slots, &cus))) return rc;
        // the equal-share plan when the uniform split grid would take more than one round of
        // resident blocks (long or ragged contexts); otherwise one block per (unit, split)
        P.dq_lead = 0;
        if (use_decode) P.pv_tiles = pl.split_len / EA_TILE;
        if (use_decode && pl.nsplit_gen >= 2 && (int64_t)pl.dq_units * pl.nsplit_gen == slots && slots > cus) {
            // exactly one round: the first wave's splits are weighted 5 against 4 (the decode
            // kernel's uniform path); the longest is at most 5 / (5 + 4 (n - 1)) of the unit's
            // tiles, plus one for the rounding
            const int64_t tt = (int64_t)pl.nsplit_gen * (pl.split_len / EA_TILE), den = 5 + 4 * (int64_t)(pl.nsplit_gen - 1);
            P.dq_lead = cus;
            P.pv_tiles = (int32_t)((5 * tt + den - 1) / den + 1);
        }
        if (use_decode && (int64_t)pl.dq_units * pl.nsplit_gen > slots) {
            const int64_t nb = std::min<int64_t>(slots, EA_DQ_MAX_BLOCKS);
            P.dq_stream = 1;
            P.nsplit = pl.nsplit;
            P.dq_units = pl.dq_units;
            P.dq_blocks = (int32_t)(nb > 0 ? nb : 1);
            P.dq_min_share = pl.dq_min_share;
            P.dq_max_tiles = pl.dq_max_tiles;
            P.dq_rec_off = pl.dq_rec_off;
            P.dq_plan = (int32_t*)(ws + pl.off_dq);
        }
    }
    auto mark = [&](int i) -> int {
        return (o->events && o->events[i]) ? herr(hipEventRecord((hipEvent_t)o->events[i], st)) : 0;
    };
    if ((rc = mark(0))) return rc;
    if (pl.prefill) {
        // int8-MFMA prefill: slicing, then one kernel that certifies and writes every row; the
        // rows it leaves go to tier 2
        if ((rc = ea_launch_prefill(P, st))) return rc;
        if ((rc = mark(1))) return rc;
        if ((rc = ea_launch_prefill_main(P, st))) return rc;
        if ((rc = mark(2))) return rc;
        if ((rc = ea_launch_prefill_combine(P, st))) return rc;
        if ((rc = mark(3))) return rc;
        if (o->tier2) {
            if ((rc = list_all(P, o, rb4 * 4 / 256 + 1, st))) return rc;
            hipLaunchKernelGGL(ea_tier2, dim3(EA_T2_BLOCKS), dim3(EA_T2_THREADS), 0, st, P);
            rc = herr(hipGetLastError());
            if (rc) return rc;
        }
        return mark(4);
    }
    // the decode kernel on uniform splits prepares its own rows' q (and clears the work list)
    if (!(use_decode && !P.dq_stream)) {
        hipLaunchKernelGGL(ea_prep, dim3(rb4 + (P.dq_stream ? 1u : 0u)), dim3(256), 0, st, P);
        rc = herr(hipGetLastError());
        if (rc) return rc;
    }
    if (pl.nseg > 0) {
        static std::once_flag once;
        static hipError_t attr_err = hipSuccess;
        std::call_once(once, [] {
            const void* fns[6] = {(const void*)ea_split<1, false>, (const void*)ea_split<2, false>,
                                  (const void*)ea_split<4, false>, (const void*)ea_split<1, true>,
                                  (const void*)ea_split<2, true>, (const void*)ea_split<4, true>};
            for (const void* f : fns) {
                hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)sizeof(SplitSmem));
                if (e != hipSuccess) attr_err = e;
            }
        });
        rc = herr(attr_err);
        if (rc) return rc;
        dim3 grid((unsigned)(pl.nseg * pl.nrb), (unsigned)pl.nsplit_gen);
        if ((rc = mark(1))) return rc;
        const dim3 blk(EA_THREADS);
        const size_t lds = sizeof(SplitSmem);
        if (use_decode) {
            if ((rc = ea_launch_decode(P, st))) return rc;
        } else if (o->timers) {
            if (pl.rb == 1) hipLaunchKernelGGL((ea_split<1, true>), grid, blk, lds, st, P);
            else if (pl.rb == 2) hipLaunchKernelGGL((ea_split<2, true>), grid, blk, lds, st, P);
            else hipLaunchKernelGGL((ea_split<4, true>), grid, blk, lds, st, P);
        } else {
            if (pl.rb == 1) hipLaunchKernelGGL((ea_split<1, false>), grid, blk, lds, st, P);
            else if (pl.rb == 2) hipLaunchKernelGGL((ea_split<2, false>), grid, blk, lds, st, P);
            else hipLaunchKernelGGL((ea_split<4, false>), grid, blk, lds, st, P);
        }
        rc = herr(hipGetLastError());
        if (rc) return rc;
    } else if ((rc = mark(1))) {
        return rc;
    }
    if ((rc = mark(2))) return rc;
    hipLaunchKernelGGL(ea_combine, dim3((unsigned)pl.rows), dim3(64), 0, st, P);
    rc = herr(hipGetLastError());
    if (rc) return rc;
    if ((rc = mark(3))) return rc;
    if (o->tier2) {
        if ((rc = list_all(P, o, rb4 * 4 / 256 + 1, st))) return rc;
        hipLaunchKernelGGL(ea_tier2, dim3(EA_T2_BLOCKS), dim3(EA_T2_THREADS), 0, st, P);
        rc = herr(hipGetLastError());
        if (rc) return rc;
    }
    return mark(4);
}

int ea_hip_attention_noalloc(const ea_geometry* g, const ea_buffers* bf, const ea_options* o, ea_stream_t stream) {
    size_t need = 0;
    int32_t ns = 0;
    int rc = ea_hip_workspace_size(g, o, &need, &ns);
    if (rc) return rc;
    if (need > (size_t)EA_NOALLOC_SCRATCH_BYTES) return -4;
    void* ws = nullptr;
    if ((rc = scratch_address(&ws))) return rc;
    return ea_hip_attention(g, bf, o, ws, (size_t)EA_NOALLOC_SCRATCH_BYTES, stream);
}

static int exact_rows_impl(const ea_geometry* g, const ea_buffers* bf, const ea_options* o, ea_stream_t stream) {
    Plan pl;
    int rc = make_plan(g, o, &pl);
    if (rc) return rc;
    if (pl.rows == 0) return ((o->alpha_bits >> 23) & 0xFF) == 0xFF ? -3 : 0;  // an empty batch
    if (!bf || !bf->q || !bf->k || !bf->v || !bf->seq_len || !bf->kv_len || !bf->out || !bf->flags) return -1;
    if (bf->tree_mask && !bf->tree_base) return -1;
    if (((o->alpha_bits >> 23) & 0xFF) == 0xFF) return -3;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e = hipStreamSynchronize(st);
    if (e != hipSuccess) return herr(e);
    std::vector<uint8_t> fl((size_t)pl.rows);
    if ((e = hipMemcpy(fl.data(), bf->flags, (size_t)pl.rows, hipMemcpyDeviceToHost)) != hipSuccess) return herr(e);
    std::vector<int64_t> todo;
    for (int64_t r = 0; r < pl.rows; ++r)
        if (fl[(size_t)r] == 1) todo.push_back(r);
    if (todo.empty()) return 0;
    Params P;
    memset(&P, 0, sizeof(P));
    P.g = *g;
    P.q = bf->q; P.k = bf->k; P.v = bf->v;
    P.seq_len = bf->seq_len; P.kv_len = bf->kv_len; P.bt = bf->block_table; P.bt_off = bf->block_table_offset;
    P.tree_mask = bf->tree_mask; P.tree_base = bf->tree_base;
    P.grp = pl.grp; P.pshift = pl.pshift; P.rows = pl.rows;
    const int d = g->head_dim, dv = g->head_dim_v, T = g->num_tokens, Hq = g->num_q_heads;
    // visible keys per listed row: the prefix plus the tree keys (vis_prefix, vis_tree_bits)
    std::vector<int64_t> nk(todo.size());
    int64_t maxk = 0;
    for (size_t i = 0; i < todo.size(); ++i) {
        const int64_t row = todo[i], b = row / ((int64_t)T * Hq), t = (row / Hq) % T, tok = b * T + t;
        int32_t L = 0, sl = 0, tb = 0;
        uint64_t m = 0;
        if ((e = hipMemcpy(&L, bf->kv_len + tok, 4, hipMemcpyDeviceToHost)) != hipSuccess) return herr(e);
        if ((e = hipMemcpy(&sl, bf->seq_len + b, 4, hipMemcpyDeviceToHost)) != hipSuccess) return herr(e);
        if (bf->tree_mask) {
            if ((e = hipMemcpy(&m, bf->tree_mask + tok, 8, hipMemcpyDeviceToHost)) != hipSuccess) return herr(e);
            if ((e = hipMemcpy(&tb, bf->tree_base + b, 4, hipMemcpyDeviceToHost)) != hipSuccess) return herr(e);
        }
        const int64_t Lc = vis_prefix(L, sl);
        nk[i] = Lc + __builtin_popcountll(bf->tree_mask ? vis_tree_bits(m, tb, Lc, sl) : 0ull);
        maxk = nk[i] > maxk ? nk[i] : maxk;
    }
    const size_t cap = (size_t)(d + maxk * (int64_t)(d + dv));
    std::vector<uint16_t> host(cap);  // before the device buffer: a throw here leaks nothing
    uint16_t* stage = nullptr;
    if ((e = hipMalloc(&stage, cap * 2)) != hipSuccess) return herr(e);
    const size_t osz = o->out_fp32 ? 4 : 2;
    int64_t fixed = 0, refused = 0, dom = 0;
    for (size_t i = 0; i < todo.size() && e == hipSuccess; ++i) {
        const int64_t row = todo[i], n = nk[i];
        const int64_t b = row / ((int64_t)T * Hq), t = (row / Hq) % T, hq = row % Hq;
        const size_t cnt = (size_t)(d + n * (int64_t)(d + dv));
        const unsigned blocks = (unsigned)std::min<size_t>((cnt + 255) / 256, 4096);
        hipLaunchKernelGGL(ea_gather_row, dim3(blocks), dim3(256), 0, st, P, row, n, stage);
        if ((e = hipGetLastError()) != hipSuccess) break;
        if ((e = hipMemcpyAsync(host.data(), stage, cnt * 2, hipMemcpyDeviceToHost, st)) != hipSuccess) break;
        if ((e = hipStreamSynchronize(st)) != hipSuccess) break;
        uint8_t res[EA_MAXDV * 4];  // dv bf16 (uint16) or fp32 (uint32) patterns, as exact_row writes them
        const int x = eax::exact_row(host.data(), d, host.data() + d, host.data() + d + n * d, n, dv, o->alpha_bits,
                                     o->out_fp32, res, nullptr);
        if (x == eax::EAX_NOMEM) {
            (void)hipFree(stage);
            return EA_ERR_HOST_MEMORY;
        }
        uint8_t flag = x == eax::EAX_OK ? 0 : 2;
        if (x != eax::EAX_OK) memset(res, 0, sizeof(res));
        fixed += x == eax::EAX_OK;
        refused += x == eax::EAX_REFUSED;
        dom += x == eax::EAX_DOMAIN;
        const int64_t obase = b * g->o_seq_stride + t * g->o_tok_stride + hq * g->o_head_stride;
        char* dst = (char*)bf->out + obase * (int64_t)osz;
        e = hipMemcpy(dst, res, (size_t)dv * osz, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(bf->flags + row, &flag, 1, hipMemcpyHostToDevice);
    }
    (void)hipFree(stage);
    if (e != hipSuccess) return herr(e);
    if (o->stats) {
        int64_t hs[16];
        if ((e = hipMemcpy(hs, o->stats, sizeof(hs), hipMemcpyDeviceToHost)) != hipSuccess) return herr(e);
        hs[13] += fixed;
        hs[14] += refused;
        hs[4] += refused + dom;
        if ((e = hipMemcpy(o->stats, hs, sizeof(hs), hipMemcpyHostToDevice)) != hipSuccess) return herr(e);
    }
    return 0;
}

int ea_hip_exact_rows(const ea_geometry* g, const ea_buffers* bf, const ea_options* o, ea_stream_t stream) {
    try {
        return exact_rows_impl(g, bf, o, stream);
    } catch (...) {  // host vectors: only an exhausted heap throws
        return EA_ERR_HOST_MEMORY;
    }
}

int ea_exact_row(const uint16_t* q, int d, const uint16_t* k, const uint16_t* v, int64_t n, int dv,
                 uint32_t alpha_bits, int fp32_out, void* out, uint32_t* t_bits, int32_t* w_m, int64_t* w_e) {
    if (!q || !out || d <= 0 || dv <= 0 || n < 0 || (n > 0 && (!k || !v))) return -1;
    eax::KeyTrace tr{t_bits, w_m, w_e};
    const int x = eax::exact_row(q, d, k, v, n, dv, alpha_bits, fp32_out ? 1 : 0, out,
                                 (t_bits || w_m || w_e) ? &tr : nullptr);
    return x == eax::EAX_NOMEM ? EA_ERR_HOST_MEMORY : x;
}

float ea_round_ratio(uint64_t a_hi, uint64_t a_lo, uint64_t b_hi, uint64_t b_lo, int E, int neg, int fp32,
                     int* overflow) {
    int ov = 0;
    const uint32_t bits = eax::round_ratio_bits(a_hi, a_lo, b_hi, b_lo, E, neg, fp32, &ov);
    if (overflow) *overflow = ov;
    const uint32_t f = fp32 ? bits : (bits << 16);
    float r;
    memcpy(&r, &f, 4);
    return r;
}

int ea_hip_kv_append(uint16_t* k_pool, uint16_t* v_pool, int64_t pool_rows, int64_t row_elems, const uint16_t* k_new,
                     const uint16_t* v_new, const int64_t* dst_rows, int64_t n, int32_t* block_table,
                     int64_t block_table_entries, const int64_t* bt_pos, const int32_t* bt_val, int64_t n_bt,
                     ea_stream_t stream) {
    if (n < 0 || n_bt < 0 || pool_rows < 0 || row_elems <= 0 || block_table_entries < 0) return -1;
    if (n > 0 && (!k_pool || !v_pool || !k_new || !v_new || !dst_rows)) return -1;
    if (n_bt > 0 && (!block_table || !bt_pos || !bt_val)) return -1;
    if (n == 0 && n_bt == 0) return 0;
    const hipStream_t st = (hipStream_t)stream;
    const bool wide = row_elems % 8 == 0 &&
                      ((uintptr_t)k_pool | (uintptr_t)v_pool | (uintptr_t)k_new | (uintptr_t)v_new) % 16 == 0;
    const int64_t row_u = wide ? row_elems / 8 : row_elems;
    const int64_t work = std::max(n * row_u, n_bt);
    const unsigned grid = (unsigned)std::min<int64_t>((work + 255) / 256, 1024);
    if (wide)
        hipLaunchKernelGGL(ea_kv_append<uint4>, dim3(grid), dim3(256), 0, st, (uint4*)k_pool, (uint4*)v_pool,
                           pool_rows, row_u, (const uint4*)k_new, (const uint4*)v_new, dst_rows, n, block_table,
                           block_table_entries, bt_pos, bt_val, n_bt);
    else
        hipLaunchKernelGGL(ea_kv_append<uint16_t>, dim3(grid), dim3(256), 0, st, k_pool, v_pool, pool_rows, row_u,
                           k_new, v_new, dst_rows, n, block_table, block_table_entries, bt_pos, bt_val, n_bt);
    return herr(hipGetLastError());
}

size_t ea_hip_kv_digits_bytes(int32_t num_seqs, int32_t num_kv_heads, int32_t tiles_per_seq) {
    if (num_seqs <= 0 || num_kv_heads <= 0 || tiles_per_seq <= 0) return 0;
    return (size_t)num_seqs * num_kv_heads * tiles_per_seq * EA_PF_TILE_BYTES;
}

int ea_hip_kv_digits_update(const ea_geometry* g, const ea_buffers* b, const int32_t* key_begin,
                            const int32_t* key_end, int32_t max_new_keys, void* kv_digits, int32_t tiles_per_seq,
                            ea_stream_t stream) {
    if (!g || !b || !b->k || !b->v || !b->seq_len || !key_begin || !key_end || !kv_digits) return -1;
    if (tiles_per_seq <= 0 || max_new_keys < 0 || g->num_seqs < 0 || g->num_kv_heads <= 0) return -1;
    if (g->head_dim != 128 || g->head_dim_v != 128) return -1;  // the digit tiles are for d = dv = 128
    if (g->page_size <= 0 || (g->page_size & (g->page_size - 1))) return -1;
    if ((int64_t)tiles_per_seq * 64 >= (1 << 30)) return -1;
    if (max_new_keys == 0 || g->num_seqs == 0) return 0;
    Params P;
    memset(&P, 0, sizeof(P));
    P.g = *g;
    P.k = b->k; P.v = b->v; P.seq_len = b->seq_len; P.bt = b->block_table; P.bt_off = b->block_table_offset;
    int ps = 0;
    while ((1 << ps) < g->page_size) ++ps;
    P.pshift = ps;
    P.nseg = g->num_seqs * g->num_kv_heads;
    P.pfkv = (uint8_t*)kv_digits;
    P.pf_ntiles = tiles_per_seq;
    P.kvd_begin = key_begin;
    P.kvd_end = key_end;
    P.kvd_span = (int32_t)(((int64_t)max_new_keys + 63) / 64 + 1);  // a key range meets at most this many tiles
    return ea_launch_kv_digits(P, (hipStream_t)stream);
}

int ea_hip_kat_weight(int64_t n, const uint32_t* t_bits, int32_t* M, int64_t* E, int32_t* status, int32_t* M2,
                      int64_t* E2, int32_t* status2, ea_stream_t stream) {
    if (n <= 0) return n < 0 ? -1 : 0;
    hipLaunchKernelGGL(ea_kat_weight, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, n, t_bits,
                       M, E, status, M2, E2, status2);
    return herr(hipGetLastError());
}

int ea_hip_kat_wave_max(int64_t nwaves, const int32_t* in, int32_t* out, ea_stream_t stream) {
    if (nwaves <= 0) return nwaves < 0 ? -1 : 0;
    hipLaunchKernelGGL(ea_kat_wave_max, dim3((unsigned)nwaves), dim3(64), 0, (hipStream_t)stream, nwaves, in, out);
    return herr(hipGetLastError());
}

int ea_hip_kat_round(int64_t n, const double* x, const double* r, int32_t fp32, uint32_t* bits, int32_t* ok,
                     ea_stream_t stream) {
    if (n <= 0) return n < 0 ? -1 : 0;
    hipLaunchKernelGGL(ea_kat_round, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, n, x, r,
                       fp32, bits, ok);
    return herr(hipGetLastError());
}

int ea_hip_kat_rn32_prod(int64_t n, const int32_t* am, const int64_t* x_hi, const uint64_t* x_lo, const int32_t* E,
                         uint32_t* bits, int32_t* status, ea_stream_t stream) {
    if (n <= 0) return n < 0 ? -1 : 0;
    hipLaunchKernelGGL(ea_kat_rn32_prod, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, n, am,
                       x_hi, x_lo, E, bits, status);
    return herr(hipGetLastError());
}

int ea_hip_kat_round_ratio(int64_t n, const uint64_t* a_hi, const uint64_t* a_lo, const uint64_t* b_hi,
                           const uint64_t* b_lo, const int32_t* E, const int32_t* neg, int32_t fp32, uint32_t* bits,
                           int32_t* overflow, ea_stream_t stream) {
    if (n <= 0) return n < 0 ? -1 : 0;
    hipLaunchKernelGGL(ea_kat_round_ratio, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, n,
                       a_hi, a_lo, b_hi, b_lo, E, neg, fp32, bits, overflow);
    return herr(hipGetLastError());
}

int ea_hip_kat_certify_quotient(int64_t n, const int64_t* cases, int32_t fp32, uint32_t* bits, int32_t* ok,
                                ea_stream_t stream) {
    if (n <= 0) return n < 0 ? -1 : 0;
    if (!cases || !bits || !ok) return -1;
    hipLaunchKernelGGL(ea_kat_certify_quotient, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       n, cases, fp32, bits, ok);
    return herr(hipGetLastError());
}

}  // extern "C"
