// Tier-1 decode kernel for d = dv = 128 on gfx950: one wave per (segment, row block, KV split).
//
// The reference runs this step as its Triton split program (src/exactattn/triton_kernels.py:
// 730-1077) over precomputed int8 slice planes (~1053 bytes per key and KV head). Here the wave
// reads the raw bf16 K/V pages (512 bytes per key and KV head) and computes in fp64, which CDNA4
// issues at the full VALU rate:
//
//   K tile  64 keys (16 KB), DMA'd by global_load_lds_dwordx4 straight into LDS (no VGPR
//           round trip), 16-byte chunks XOR-swizzled by key so per-key reads are conflict-free;
//           double-buffered, tile i+1 in flight while tile i is processed.
//   S       lane = key: two fp64 FMA chains per row over the 128 dims, q as SGPR operands
//           (scalar loads of the fp64 q: on uniform splits wave A converts the block's bf16 q
//           rows itself before the first barrier, which takes the prep kernel off the step;
//           the stream plan keeps the prep kernel). Rounding error of the chains is bounded
//           by 66 u sum_b |q_b|_1 |k_b|_inf over four 32-dim blocks (|k_b|_inf from v_max3_f32
//           on the fp32 patterns the conversion makes anyway).
//   B       lane = key, every row: certified t = RN32(alpha s) from the interval, RN24(2^t)
//           from the fp64 tables; pairs the interval cannot decide take the exact TwoSum path.
//           Running per-row reference exponent from a DPP wave max; weights to LDS.
//   P       lane = (key group g, 8 channels): V rows of 4 keys per dwordx4 load (1 KB per
//           instruction, coalesced, page base on the scalar unit), double-buffered in VGPRs;
//           exact products omega*v summed by FMA.
// The epilogue reduces the 4 key groups and writes the split partial in the layout the combine
// kernel reads (R, n, Z, N[dv] per split and row; max |v| per channel per row block).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "ea_params.h"

using namespace ea;

namespace {

constexpr int DT = 64;  // keys per tile = lanes

// Rows [0, RA) of a block are certified by wave A, rows [RA, RB) by wave B (from scores and bounds
// wave A hands over), so the two waves' instruction streams per tile are about equally long.
template <int RB>
constexpr int rows_a() { return (RB + 1) / 2; }

template <int RB>
struct DecodeSmem {
    static constexpr int RA = rows_a<RB>(), RBB = RB - RA > 0 ? RB - RA : 1;
    uint4 K[2][DT * 16];     // 2 x 16 KB K tiles; reused by the epilogue reduction
    double w[2][DT][RA];     // wave A's weights of a tile, [key][row], double-buffered between the waves
    double2 sb[2][DT][RBB];  // (score, error bound) of wave B's rows; wave B overwrites .x with the weight
    double sc[2][RA];        // rescale of wave A's rows' running P.V sums before that tile
    double T1[256], T2[256];
    // uniform splits, computed by wave A: each row's q NaN/inf flag and its per-32-dim-block
    // |q| bounds (the score bound reads them here: two rows share a line of the qn array, and a
    // scalar load of it could hold another block's row from before that block stored it)
    double qnb[RB][4];
    int qbad[RB];
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

// s_waitcnt vmcnt(n), expcnt/lgkmcnt untouched (gfx9 encoding: vmcnt[3:0], expcnt[6:4],
// lgkmcnt[11:8], vmcnt[5:4] in bits 15:14)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ float absf(float x) { return __builtin_fabsf(x); }

}  // namespace

template <int RB, int PGL, bool STREAM>
__device__ __forceinline__ void decode_body(Params P) {
    static_assert(RB == 1 || RB == 2, "1- or 2-row blocks (two waves per SIMD)");
    extern __shared__ __align__(16) unsigned char smem_raw[];
    DecodeSmem<RB>& S = *reinterpret_cast<DecodeSmem<RB>*>(smem_raw);

    // the exp2 tables go to LDS from wave A, their global loads issued just before its first K
    // DMA and their LDS writes after it (the two latencies overlap); first piece only
    bool tables_due = true;
    // the decode kernel takes every row of the problem: one add for the whole grid
    if constexpr (STREAM)
        if (threadIdx.x == 0 && P.stats && blockIdx.x == 0) atomicAdd((unsigned long long*)&P.stats[9], (unsigned long long)P.rows);

    // One piece: keys [kA, kB) of unit `item` (segment, row block), clipped to the unit's visible
    // end, as partial slot `split`.
    auto piece = [&](const int item, const int split, const int kA, const int kB) __attribute__((always_inline)) {
    // lane-derived values are recomputed from an opaque copy of the lane index in every piece, so
    // that none of them is hoisted out of the piece loop and kept live across it
    int lane_ = (int)(threadIdx.x & 63);
    if constexpr (STREAM) asm volatile("" : "+v"(lane_));
    const int lane = lane_;
    const int g = lane >> 4, c8 = lane & 15;
    const int seg = item / P.nrb, rbk = item % P.nrb;
    const int Hkv = P.g.num_kv_heads;
    const int b = seg / Hkv;
    const int hk = seg % Hkv;
    const int row0 = rbk * P.rb;
    const int nrow = min(RB, P.r_seg - row0);
    cint_t* kvl4 = (cint_t*)P.kv_len;
    cint_t* qinfo4 = (cint_t*)P.qinfo;
    cdouble_t* qn4 = (cdouble_t*)P.qn;
    // the fp64 q rows (written in this kernel on uniform splits): every read goes through this
    // base, which is handed out again by an empty asm after the barrier that follows the writes,
    // so no load through it can be scheduled before them
    cdouble_t* q64b = (cdouble_t*)P.q64;
    // rows of the block (a short block repeats its last row; repeats are never written). Key
    // positions, lengths and row indices fit 31 bits (checked by the launcher).
    int grow[RB];
    int kvl[RB];
    uint64_t tmk[RB];
    int rflag[RB];
    int kend = 0;
    int tb = 0;
    if (P.tree_mask) tb = ((cint_t*)P.tree_base)[b];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        int lr = row0 + min(r, nrow - 1);
        int t = lr / P.grp, gi = lr % P.grp;
        grow[r] = (int)row_index(P, b, t, hk * P.grp + gi);
        int tok = b * P.g.num_tokens + t;
        kvl[r] = kvl4[tok];
        tmk[r] = P.tree_mask ? ((const uint64_t __attribute__((address_space(4)))*)P.tree_mask)[tok] : 0ull;
        int e = kvl[r];
        if (tmk[r]) e = max(e, tb + 64 - (int)__clzll(tmk[r]));
        kend = max(kend, e);
        if constexpr (STREAM) rflag[r] = qinfo4[grow[r] * 5 + 4] ? 1 : 0;
        else rflag[r] = 0;  // set once wave A has converted the rows' q
    }
    const int slen = ((cint_t*)P.seq_len)[b];
    if (kend > slen) kend = slen;
    const int k0 = kA;
    const int k1 = min(kB, kend);
    const int64_t pbase = (int64_t)split * P.rows;
    cint_t* btb = (cint_t*)P.bt + (P.bt ? (P.bt_off ? P.bt_off[b] : (int64_t)b * P.g.block_table_stride) : 0);
    const int pshift = P.pshift;
    const int pmask = (1 << pshift) - 1;
    // byte strides; the slot part of an address goes into the 32-bit soffset
    const int64_t kps2 = 2 * P.g.k_page_stride, vps2 = 2 * P.g.v_page_stride;
    const int kss2 = (int)(2 * P.g.k_slot_stride), vss2 = (int)(2 * P.g.v_slot_stride);
    const char* kh = (const char*)(P.k + (int64_t)hk * P.g.k_head_stride);
    const char* vh = (const char*)(P.v + (int64_t)hk * P.g.v_head_stride);
    // per-lane byte offsets inside a 4-key group: K lane (g, p) brings chunk p ^ ((4j + g) & 15)
    // of key 4j + g (the XOR depends on j only through j & 3); V lane (g, c8) channels 8 c8 ..
    int koff[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) koff[jj] = g * kss2 + ((c8 ^ ((4 * jj + g) & 15)) << 4);
    const int voff = g * vss2 + (c8 << 4);

    // Group j of the tile at n0 holds keys n0+4j .. n0+4j+3, all in one page (page size >= 4 and
    // n0 % 64 == 0). Pages are looked up every PGL keys (PGL <= page size, or the whole
    // sequence without a block table); inside a lookup interval the slot advances by 4 keys per
    // group. Lanes whose key is at or past k1 get the offset EA_OOB: the buffer unit's range
    // check (offset >= num_records) returns zeros without a memory access, so every tile issues
    // exactly 16 K and 16 V instructions with no branches. Lookup indices are clamped to k1 - 1
    // so the block table is never read past the sequence.
    constexpr int EA_OOB = (int)0x80000000u;
    auto page_rs = [&](int n, const char* head, int64_t ps2, int* slot) __attribute__((always_inline)) {
        int64_t pg;
        const int nc = min(n, k1 - 1);
        if (P.bt) {
            pg = btb[nc >> pshift];
            *slot = n & pmask;
        } else {
            pg = b;
            *slot = n;
        }
        return __builtin_amdgcn_make_buffer_rsrc((void*)(head + pg * ps2), (short)0, 0x7FFFFFFF, 0x00020000);
    };
    // K tile at n0 -> LDS buffer `buf`: instruction j writes the 1 KB of keys 4j..4j+3
    auto issue_k = [&](int n0, int buf) __attribute__((always_inline)) {
        __amdgpu_buffer_rsrc_t rs;
        int slot = 0;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int nj = n0 + 4 * j;
            if ((4 * j) % PGL == 0) rs = page_rs(nj, kh, kps2, &slot);
            const int sl = slot + (4 * j) % PGL;
            const int off = (nj + g < k1) ? koff[j & 3] : EA_OOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)&S.K[buf][j * 64], 16, off, sl * kss2, 0, 2);
        }
    };
    auto issue_v = [&](int n0, u32x4 (&vr)[16], double d0, double d1) __attribute__((always_inline)) {
        __amdgpu_buffer_rsrc_t rs;
        int slot = 0;
        int vo = voff;
        asm volatile("" : "+v"(vo) : "v"(d0), "v"(d1));
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int nj = n0 + 4 * j;
            if ((4 * j) % PGL == 0) rs = page_rs(nj, vh, vps2, &slot);
            const int sl = slot + (4 * j) % PGL;
            const int off = (nj + g < k1) ? vo : EA_OOB;
            vr[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, sl * vss2, 2);
        }
    };

    const double alpha = P.alpha;
    const double gam = 66.0 * 0x1p-53 * (1.0 + 0x1p-20);
    const int ntiles = (k1 > k0) ? (int)((k1 - k0 + DT - 1) / DT) : 0;
    // Both roles run ntiles + 1 loop iterations with one barrier each (and the prologue barrier):
    // iteration it has wave A publish the weights of tile it, wave B consume those of tile it - 1.
    const int role = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    constexpr int RA = rows_a<RB>();

    // Per-row certification state; each wave keeps the rows it certifies (A: [0, RA), B: [RA, RB)).
    int Rrun[RB];
    double zacc[RB];
    int nvis[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        Rrun[r] = INT_MIN;
        zacc[r] = 0.0;
        nvis[r] = 0;
    }
    // Certified weight of row r at key n = lane's key, from the fp64 score s and its error bound
    // del: t = RN32(alpha s) certified from the interval (pairs it cannot decide are redone exactly
    // by `exact`, which returns the TwoSum sum, its error sum and the sum of |errors| of the
    // products of q row r and key n), w = RN24(2^t). Advances the row's running reference exponent
    // (a DPP wave max), Z sum, visible count and flag; returns the weight scaled to the reference
    // exponent, and in *fout the wave-uniform rescale of the row's running sums.
    auto certify = [&](int r, int n, double s, double del, auto&& exact, double* fout) __attribute__((always_inline)) {
        const int ti = n - tb;
        const bool vis = (n < k1) && (n < kvl[r] || (ti >= 0 && ti < 64 && ((tmk[r] >> ti) & 1)));
        int32_t M = 1 << 23, E = -23;
        int why = 0;  // 1 score not certified, 2 weight not certified, 3 weight out of range
        bool slow = false;
        if (vis && !rflag[r]) {
            uint32_t tbits = 0;
            int ls = isfinite(s) ? logit_cert(alpha, s, 0.0, del, &tbits) : 3;
            if (ls == 3 && isfinite(s)) {
                // exact path: every product separately, TwoSum-accumulated
                slow = true;
                double ss = 0.0, es = 0.0, ea = 0.0;
                exact(r, n, ss, es, ea);
                ls = (ss == 0.0 && es == 0.0 && ea == 0.0) ? 1 : logit_cert(alpha, ss, es, ea * 0x1p-44, &tbits);
            }
            if (ls == 2 || ls == 3) {
                why = 1;
            } else if (ls == 0) {
                int ws = weight_f64(tbits, S.T1, S.T2, &M, &E);
                if (ws) {
                    int32_t M2 = 0;
                    int64_t E2 = 0;
                    if (weight_wide(tbits, &M2, &E2) == 0 && E2 > -(1LL << 30) && E2 < (1LL << 30)) {
                        M = M2;
                        E = (int32_t)E2;
                    } else {
                        why = 2;
                    }
                }
            }
        }
        if (P.stats) {
            const uint64_t b1 = __ballot(why == 1), b2 = __ballot(why == 2), b3 = __ballot(slow);
            if (lane == 0 && b1) atomicAdd((unsigned long long*)&P.stats[5], (unsigned long long)__popcll(b1));
            if (lane == 0 && b2) atomicAdd((unsigned long long*)&P.stats[6], (unsigned long long)__popcll(b2));
            if (lane == 0 && b3) atomicAdd((unsigned long long*)&P.stats[8], (unsigned long long)__popcll(b3));
        }
        const bool live = vis && why == 0;
        const int tmax = wave_max_dpp(live ? E + 23 : INT_MIN);
        const int Rnew = max(Rrun[r], tmax);
        const bool far = live && (E - Rnew < -1000);
        if (__ballot(why != 0 || far)) rflag[r] = 1;
        double f = 1.0;  // rescale of the running sums to the new reference exponent
        if (Rrun[r] != INT_MIN && Rnew != Rrun[r]) {
            const int dsh = Rrun[r] - Rnew;
            if (dsh < -900) rflag[r] = 1;
            f = ldexp(1.0, max(dsh, -1000));
            zacc[r] *= f;
        }
        Rrun[r] = Rnew;
        double om = (live && !far) ? ldexp((double)M, E - Rnew) : 0.0;
        if (rflag[r]) om = 0.0;
        zacc[r] += om;
        nvis[r] += vis ? 1 : 0;
        *fout = f;
        return om;
    };
    // q row r's fp64 values (the prep kernel's, or on uniform splits wave A's), for the exact path
    auto qrow64 = [&](int r) __attribute__((always_inline)) { return q64b + (int64_t)grow[r] * EA_MAXD; };

    // R, Z and the visible count (-1: flagged) of rows [r0, r1) into the split partial
    auto publish_rows = [&](int r0, int r1) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            if (r < r0 || r >= r1) continue;
            const double zs = wave_sum(zacc[r]);
            const int ns = wave_sum_i(nvis[r]);
            if (lane == 0 && r < nrow) {
                const int64_t o = pbase + grow[r];
                P.pR[o] = Rrun[r];
                P.pZ[o] = zs;
                P.pn[o] = rflag[r] ? -1 : ns;
            }
        }
    };

    // exact products of q row r and key n, the key read from the cache (its LDS tile is being
    // refilled by then: wave B's pairs, and wave A's with the equal-share plan); only pairs the
    // fp64 interval cannot decide come here
    auto exact_global = [&](int r, int n, double& ss, double& es, double& ea) __attribute__((always_inline)) {
        const int64_t pg = P.bt ? (int64_t)btb[n >> pshift] : (int64_t)b;
        const int sl = P.bt ? (n & pmask) : n;
        const uint4* kp = (const uint4*)(kh + pg * kps2 + (int64_t)sl * kss2);
        cdouble_t* qr = qrow64(r);
        for (int c = 0; c < 16; ++c) {
            const uint4 kv = kp[c];
            const uint32_t wd[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                double e0, e1;
                ss = two_sum(ss, qr[8 * c + 2 * j] * bf16lo_f64(wd[j]), &e0);
                ss = two_sum(ss, qr[8 * c + 2 * j + 1] * bf16hi_f64(wd[j]), &e1);
                es += e0 + e1;
                ea += fabs(e0) + fabs(e1);
            }
        }
    };

    if (role == 0) {
        // ============ wave A: K tiles, scores, certified logits and weights of rows [0, RA)
        // uniform splits: this block converts its rows' q (the prep kernel's work for these rows;
        // every split's block stores the same values), the loads issued before the first K DMA
        uint32_t qx[RB][2];
        if constexpr (!STREAM) {
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const int64_t row = grow[r];
                const int64_t bb = row / ((int64_t)P.g.num_tokens * P.g.num_q_heads);
                const int tt = (int)((row / P.g.num_q_heads) % P.g.num_tokens), hq = (int)(row % P.g.num_q_heads);
                const uint16_t* qr = P.q + bb * P.g.q_seq_stride + (int64_t)tt * P.g.q_tok_stride + (int64_t)hq * P.g.q_head_stride;
                qx[r][0] = qr[2 * lane];
                qx[r][1] = qr[2 * lane + 1];
            }
        }
        if (tables_due) {
            uint64_t tb1[4], tb2[4];
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                tb1[h] = EA_T1_BITS[lane + 64 * h];
                tb2[h] = EA_T2_BITS[lane + 64 * h];
            }
            if (ntiles > 0) issue_k(k0, 0);
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                S.T1[lane + 64 * h] = u64_as_f64(tb1[h]);
                S.T2[lane + 64 * h] = u64_as_f64(tb2[h]);
            }
            tables_due = false;
        } else if (ntiles > 0) {
            issue_k(k0, 0);
        }
        if constexpr (!STREAM) {
            double qb = 0.0;
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                if (r >= nrow) {  // a repeat of the last row: its flag and bounds
                    rflag[r] = rflag[r - 1];
                } else {
                    rflag[r] = prep_row_store(P, grow[r], lane, qx[r][0], qx[r][1], &qb);
                    if (lane == 0) S.qbad[r] = rflag[r];
                }
                if ((lane & 15) == 0) S.qnb[r][lane >> 4] = qb;
            }
            // the step's first kernel on this path clears the tier-2 work list and chunk counts
            if (item == 0 && split == 0 && lane <= EA_T2_BLOCKS) P.wl_cnt[lane] = 0;
            wait_vm<0>();  // the q stores are complete before the barrier
        }
        __syncthreads();  // tables visible
        asm volatile("" : "+s"(q64b));
        for (int it = 0; it <= ntiles; ++it) {
            if (it < ntiles) {
                const int buf = it & 1;
                const int n0 = k0 + it * DT;
                // K(it+1) into the buffer S(it-1) read (with the equal-share plan it was issued right
                // after the scores of tile it-1, K(1) here); K(it) has landed once only K(it+1)'s
                // 16 instructions may be outstanding
                if constexpr (STREAM) {
                    if (it == 0 && ntiles > 1) issue_k(k0 + DT, 1);
                } else {
                    if (it + 1 < ntiles) issue_k(n0 + DT, buf ^ 1);
                }
                if (it + 1 < ntiles) {
                    wait_vm<16>();
                } else {
                    wait_vm<0>();
                }

        // ---- S: lane = key, fp64 FMA chains (q through the scalar cache)
            double a0[RB], a1[RB];
            float km[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    #pragma unroll
            for (int r = 0; r < RB; ++r) a0[r] = a1[r] = 0.0;
            {
                // q (fp64, prep kernel) comes through the scalar cache in 4-dim halves, two halves
                // ahead of use, ping-pong between two SGPR sets. The base of the loads for half h+2 is
                // an opaque zero that consumes both FMA chains after half h: the compiler can neither
                // hoist all 128 x RB q values (they fit no register file) nor delay one chain and keep
                // its q values alive. The loads stay ordinary scalar loads (compiler lgkmcnt
                // accounting intact).
                double qA[RB][4], qB[RB][4];
                typedef const double* dptr;
                dptr qrow[RB];
    #pragma unroll
                for (int r = 0; r < RB; ++r) qrow[r] = (const double*)q64b + (int64_t)grow[r] * EA_MAXD;
                // hands out copies of the row pointers that the compiler cannot see through
                auto gate = [&](dptr (&o)[RB]) __attribute__((always_inline)) {
                    if constexpr (RB == 1) {
                        asm volatile("s_mov_b64 %0, %1" : "=&s"(o[0]) : "s"(qrow[0]), "v"(a0[0]), "v"(a1[0]));
                    } else {
                        asm volatile("s_mov_b64 %0, %2\n\ts_mov_b64 %1, %3"
                                     : "=&s"(o[0]), "=&s"(o[1])
                                     : "s"(qrow[0]), "s"(qrow[1]), "v"(a0[0]), "v"(a1[0]), "v"(a0[1]), "v"(a1[1]));
                    }
                };
                auto qload = [&](int h, double (&qv)[RB][4]) __attribute__((always_inline)) {
                    dptr o[RB];
                    gate(o);
    #pragma unroll
                    for (int r = 0; r < RB; ++r) {
                        cdouble_t* q4 = (cdouble_t*)o[r];
    #pragma unroll
                        for (int i = 0; i < 4; ++i) qv[r][i] = q4[4 * h + i];
                    }
                };
                qload(0, qA);
                qload(1, qB);
                double kf[8];
                auto half = [&](int h, double (&qc)[RB][4]) __attribute__((always_inline)) {
                    __builtin_amdgcn_sched_barrier(0);
                    const int c = h >> 1;
                    if ((h & 1) == 0) {
                        const uint4 kv = S.K[buf][lane * 16 + (c ^ (lane & 15))];
                        const uint32_t kd[4] = {kv.x, kv.y, kv.z, kv.w};
    #pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const float lo = __uint_as_float(kd[j] << 16), hi = __uint_as_float(kd[j] & 0xFFFF0000u);
                            km[c >> 2] = fmaxf(fmaxf(km[c >> 2], absf(lo)), absf(hi));
                            kf[2 * j] = (double)lo;
                            kf[2 * j + 1] = (double)hi;
                        }
                    }
                    const int o = 4 * (h & 1);
    #pragma unroll
                    for (int r = 0; r < RB; ++r) {
                        a0[r] = __fma_rn(qc[r][0], kf[o + 0], a0[r]);
                        a1[r] = __fma_rn(qc[r][1], kf[o + 1], a1[r]);
                        a0[r] = __fma_rn(qc[r][2], kf[o + 2], a0[r]);
                        a1[r] = __fma_rn(qc[r][3], kf[o + 3], a1[r]);
                    }
                    if (h + 2 < 32) qload(h + 2, qc);
                };
    #pragma unroll
                for (int h = 0; h < 32; h += 2) {
                    half(h, qA);
                    half(h + 1, qB);
                }
            }

            // ---- equal-share plan: K(it+2) into the buffer the scores just read (their LDS reads
            // are complete), so it loads during this tile's certification. Measured: C5 decode
            // kernel -2.5%; the uniform grid (C2) +1%, so it keeps the issue at the next iteration.
            if constexpr (STREAM) {
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
                if (it + 2 < ntiles) issue_k(n0 + 2 * DT, buf);
            }
            // ---- B: lane = key; rows [0, RA) certified here, the scores and bounds of rows
            // [RA, RB) handed to wave B
            __builtin_amdgcn_sched_barrier(0);
            const int n = n0 + lane;
            // exact products of q row r and this lane's key, from the K tile in LDS (the uniform
            // grid: the buffer is not refilled before the next iteration)
            auto exact_lds = [&](int r, int, double& ss, double& es, double& ea) __attribute__((always_inline)) {
                cdouble_t* qr = qrow64(r);
                for (int c = 0; c < 16; ++c) {
                    const uint4 kv = S.K[buf][lane * 16 + (c ^ (lane & 15))];
                    const uint32_t wd[4] = {kv.x, kv.y, kv.z, kv.w};
    #pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        double e0, e1;
                        ss = two_sum(ss, qr[8 * c + 2 * j] * bf16lo_f64(wd[j]), &e0);
                        ss = two_sum(ss, qr[8 * c + 2 * j + 1] * bf16hi_f64(wd[j]), &e1);
                        es += e0 + e1;
                        ea += fabs(e0) + fabs(e1);
                    }
                }
            };
    #pragma unroll
            for (int r = 0; r < RB; ++r) {
                __builtin_amdgcn_sched_barrier(0);  // one row at a time (bounded live temporaries)
                const double s = a0[r] + a1[r];
                double qn_[4];
    #pragma unroll
                for (int i = 0; i < 4; ++i) qn_[i] = STREAM ? qn4[grow[r] * 4 + i] : S.qnb[r][i];
                const double bnd = __fma_rn(qn_[0], (double)km[0],
                                    __fma_rn(qn_[1], (double)km[1], __fma_rn(qn_[2], (double)km[2], qn_[3] * (double)km[3])));
                const double del = gam * bnd * (1.0 + 0x1p-40) + 0x1p-1060;
                if (r >= RA) {
                    S.sb[buf][lane][r - RA] = make_double2(s, del);
                    continue;
                }
                double f;
                double om;
                if constexpr (STREAM) om = certify(r, n, s, del, exact_global, &f);
                else om = certify(r, n, s, del, exact_lds, &f);
                if (lane == 0) S.sc[buf][r] = f;
                S.w[buf][lane][r] = om;
            }
                }
            __syncthreads();  // weights of tile it published; wave B is done with tile it - 1
        }
        if constexpr (!STREAM)
            if (lane == 0 && P.stats && item == 0 && split == 0)
                atomicAdd((unsigned long long*)&P.stats[9], (unsigned long long)P.rows);
        publish_rows(0, RA);
    } else {
        // ============ wave B: V tiles (double-buffered in VGPRs) and the P.V sums
        double pacc[RB][8];
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int c = 0; c < 8; ++c) pacc[r][c] = 0.0;
        // max |v| over this lane's 8 channels and keys (a per-channel bound only needs to be >=
        // the channel's own maximum)
        float vmx = 0.0f;
        u32x4 vA[16], vB[16];
        if (ntiles > 0) {
            issue_v(k0, vA, 0.0, 0.0);
            issue_v(k0 + DT, vB, 0.0, 0.0);
        }
        // P of tile t with its V in vr; then V(t+2) into vr
        auto pv = [&](int t, u32x4 (&vr)[16]) __attribute__((always_inline)) {
            const int buf = t & 1;
            // rows [RA, RB) of tile t: certified here (lane = key) while V(t) is still landing;
            // the weights replace the scores in LDS for the P.V below
            if constexpr (RB > RA) {
                const int n = k0 + t * DT + lane;
#pragma unroll
                for (int r = RA; r < RB; ++r) {
                    __builtin_amdgcn_sched_barrier(0);
                    const double2 sd = S.sb[buf][lane][r - RA];
                    double f;
                    const double om = certify(r, n, sd.x, sd.y, exact_global, &f);
                    if (f != 1.0) {
#pragma unroll
                        for (int c = 0; c < 8; ++c) pacc[r][c] *= f;
                    }
                    S.sb[buf][lane][r - RA].x = om;
                }
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's weights are in LDS
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
            // V loads complete in issue order: V(t) has landed once only V(t+1)'s 16 instructions
            // may be outstanding
            wait_vm<16>();
#pragma unroll
            for (int r = 0; r < RA; ++r) {
                const double f = S.sc[buf][r];
                if (f != 1.0) {
#pragma unroll
                    for (int c = 0; c < 8; ++c) pacc[r][c] *= f;
                }
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int kk = 4 * j + g;
                double om[RB];
#pragma unroll
                for (int r = 0; r < RB; ++r) om[r] = r < RA ? S.w[buf][kk][r] : S.sb[buf][kk][r - RA].x;
                const uint32_t vd[4] = {vr[j].x, vr[j].y, vr[j].z, vr[j].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float lo = __uint_as_float(vd[q] << 16), hi = __uint_as_float(vd[q] & 0xFFFF0000u);
                    vmx = fmaxf(fmaxf(vmx, absf(lo)), absf(hi));
                    const double dlo = (double)lo, dhi = (double)hi;
#pragma unroll
                    for (int r = 0; r < RB; ++r) {
                        pacc[r][2 * q] = __fma_rn(om[r], dlo, pacc[r][2 * q]);
                        pacc[r][2 * q + 1] = __fma_rn(om[r], dhi, pacc[r][2 * q + 1]);
                    }
                }
                // zero-instruction fence: every sum and the next group's V registers count as
                // rewritten here, so groups stay in order (otherwise the compiler runs each sum's
                // chain over all 16 groups, which needs every group's converted V at once)
#pragma unroll
                for (int r = 0; r < RB; ++r)
                    asm volatile("" : "+v"(pacc[r][0]), "+v"(pacc[r][1]), "+v"(pacc[r][2]), "+v"(pacc[r][3]),
                                 "+v"(pacc[r][4]), "+v"(pacc[r][5]), "+v"(pacc[r][6]), "+v"(pacc[r][7]));
                if (j + 1 < 16) asm volatile("" : "+v"(vr[j + 1]), "+v"(vmx));
            }
            // V(t+2) into vr, issued only after the last sums of tile t (its offsets depend on them)
            issue_v(k0 + (t + 2) * DT, vr, pacc[0][0], pacc[RB - 1][7]);
        };
        // Barriers pair one to one with wave A's ntiles + 2: the prologue barrier, then one before
        // each tile (its weights are published by then) and one after the last. Straight-line
        // pairs keep vA and vB free of merges (no register copies).
        __syncthreads();  // prologue barrier (tables visible)
        asm volatile("" : "+s"(q64b));
        if constexpr (!STREAM)
#pragma unroll
            for (int r = RA; r < RB; ++r) rflag[r] = S.qbad[min(r, nrow - 1)];
        int t = 0;
        for (; t + 1 < ntiles; t += 2) {
            __syncthreads();
            pv(t, vA);
            __syncthreads();
            pv(t + 1, vB);
        }
        if (t < ntiles) {
            __syncthreads();
            pv(t, vA);
        }
        __syncthreads();  // barrier ntiles + 1: wave A runs one loop iteration past its last tile
        publish_rows(RA, RB);
        // reduce the 4 key groups (lanes 16 apart) through LDS; the K buffers are free once the
        // loop's last barrier has passed
        double* red = reinterpret_cast<double*>(&S.K[0][0]);  // [g][r][128]: 4 * RB KB <= 16 KB
        float* vred = reinterpret_cast<float*>(&S.K[1][0]);   // [g][16]
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int c = 0; c < 8; ++c) red[(g * RB + r) * 128 + 8 * c8 + c] = pacc[r][c];
        vred[g * 16 + c8] = vmx;
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes done
        __builtin_amdgcn_wave_barrier();
        for (int x = lane; x < nrow * 128; x += 64) {
            const int r = x >> 7, c = x & 127;
            double sum = red[(0 * RB + r) * 128 + c] + red[(1 * RB + r) * 128 + c];
            sum += red[(2 * RB + r) * 128 + c] + red[(3 * RB + r) * 128 + c];
            int64_t gr = 0;
#pragma unroll
            for (int rr = 0; rr < RB; ++rr)
                if (rr == r) gr = grow[rr];
            P.pN[(pbase + gr) * 128 + c] = sum;
        }
        for (int c = lane; c < 128; c += 64) {
            const int q = c >> 3;
            const float m = fmaxf(fmaxf(vred[q], vred[16 + q]), fmaxf(vred[32 + q], vred[48 + q]));
            P.pV[(((int64_t)split * P.nseg + seg) * P.nrb + rbk) * 128 + c] = m;
        }
    }
    };

    if constexpr (!STREAM) {
        // uniform splits: block (unit, split) takes keys [split split_len, (split + 1) split_len)
        // The hardware deals consecutive workgroups to the 8 XCDs in turn, and each XCD has its own
        // L2. A segment's row blocks (units seg * nrb .. seg * nrb + nrb - 1) read the same K/V
        // tiles, so they are placed 8 block indices apart, all on one XCD and dispatched close
        // together: block x runs unit ((x / 8) / nrb * 8 + x % 8) * nrb + (x / 8) % nrb (a
        // permutation of the units when nseg % 8 == 0; units % 8 == 0 keeps the split rows
        // aligned). Measured on GQA 4 and 8 decode and 4-token steps: 5-17% faster, same bits.
        int k0 = (int)blockIdx.y * P.split_len, k1 = k0 + P.split_len;
        if (P.dq_lead > 0) {
            // one full round of resident blocks: the first dq_lead blocks in dispatch order (one
            // per CU) run about 1.2x faster than the later ones (measured on C2: 80 against
            // 97-100 us with equal splits, whichever key range they take), so the unit's splits
            // among them take weight 5 and the others 4, cut in whole tiles (C2: 19, 15, 15, 15)
            const int U = (int)gridDim.x, n = (int)gridDim.y, x = (int)blockIdx.x, y = (int)blockIdx.y;
            const int nf = min(n, max(0, (P.dq_lead - x + U - 1) / U));  // splits y * U + x < dq_lead
            const int64_t tt = (int64_t)n * (P.split_len / DT), wt = 5 * nf + 4 * (n - nf);
            auto bound = [&](int yy) {
                const int64_t w = 5 * min(yy, nf) + 4 * max(0, yy - nf);
                return (int)((tt * w + wt / 2) / wt) * DT;
            };
            k0 = bound(y);
            k1 = bound(y + 1);
        }
        int item = (int)blockIdx.x;
        if (P.nrb > 1 && (P.nseg & 7) == 0) {
            const int lo = item & 7, hi = item >> 3;
            item = ((hi / P.nrb) * 8 + lo) * P.nrb + hi % P.nrb;
        }
        piece(item, (int)blockIdx.y, k0, k1);
        return;
    }
    // Block g's share of the step's tiles (the plan the prep kernel's planner block wrote): its
    // intersections with the units, in unit order, one piece each. The first comes from the
    // block's record (unit, S_u, S_(u+1), share) in one load.
    // Each XCD takes a contiguous eighth of the shares (share g runs on workgroup (g % (G/8)) * 8 +
    // g / (G/8)) when units span fewer than 8 shares on average: a segment's row-block units are
    // then neighbours on one XCD's L2. Units of 8 or more shares already put the same tiles of
    // neighbouring units 8 workgroups apart, on one XCD, and measured 3-5% slower remapped.
    int gb = (int)blockIdx.x;
    if (P.nrb > 1 && (P.dq_blocks & 7) == 0 && (int64_t)P.dq_units * 8 > P.dq_blocks)
        gb = (gb & 7) * (P.dq_blocks >> 3) + (gb >> 3);
    const int4 rec = ((const int4*)(P.dq_plan + P.dq_rec_off))[gb];
    const int W = P.dq_plan[0];
    int u = rec.x;
    const int share = rec.w;
    if (u >= P.dq_units || share <= 0) return;  // past the last share: no tile
    int start = gb * share;  // < W < 2^30
    const int end = min(start + share, W);
    {
        // the first piece, straight-line: a share inside one unit, the usual case, ends here
        const int su = rec.y, eu = rec.z;
        const int slot = gb - su / share;  // < nsplit: share >= dq_min_share
        if (slot < P.nsplit) piece(u, slot, (start - su) * DT, (min(end, eu) - su) * DT);
        start = min(end, eu);
        ++u;
    }
    // a share that crosses unit boundaries: one piece per further unit it reaches
    const int32_t* Su = P.dq_plan + 2;
    while (start < end && u < P.dq_units) {
        const int su = Su[u], eu = Su[u + 1];
        if (eu > start) {
            const int slot = gb - su / share;
            __syncthreads();  // the previous piece's LDS reads (K buffers, epilogue) are done
            if (slot < P.nsplit) piece(u, slot, (start - su) * DT, (min(end, eu) - su) * DT);
            start = min(end, eu);
        }
        ++u;
    }
}

// Launches the decode kernel when the geometry allows it; returns 1 if launched, 0 if the caller
// must use the general split kernel, or a negative HIP error code.
namespace {
// Uniform splits: one block per (unit, split). Two waves per SIMD for the 1- and 2-row blocks.
template <int RB, int PGL>
__global__ void __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(2, 2))) ea_decode(Params P) {
    decode_body<RB, PGL, false>(P);
}

// The equal-share plan: one block per share, one piece per unit the share reaches. The piece
// loop adds a few live registers; two waves per SIMD are kept for the 1- and 2-row blocks (the
// rare exact paths then reload a few values from scratch).
template <int RB, int PGL>
__global__ void __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(2, 2)))
ea_decode_stream(Params P) {
    decode_body<RB, PGL, true>(P);
}

template <int RB, bool ST>
const void* decode_fn(int pgl) {
    if constexpr (ST) {
        if (pgl == 4) return (const void*)ea_decode_stream<RB, 4>;
        if (pgl == 16) return (const void*)ea_decode_stream<RB, 16>;
        return (const void*)ea_decode_stream<RB, 64>;
    } else {
        if (pgl == 4) return (const void*)ea_decode<RB, 4>;
        if (pgl == 16) return (const void*)ea_decode<RB, 16>;
        return (const void*)ea_decode<RB, 64>;
    }
}
}  // namespace

int ea::ea_decode_eligible(const Params& P) {
    const ea_geometry& g = P.g;
    if (g.head_dim != 128 || g.head_dim_v != 128) return 0;
    if (P.bt && P.pshift < 2) return 0;
    if (P.rb != 1 && P.rb != 2) return 0;
    // 16-byte alignment of every K/V row start (dwordx4 loads)
    if (((uintptr_t)P.k | (uintptr_t)P.v) & 15) return 0;
    if ((g.k_page_stride | g.k_slot_stride | g.k_head_stride | g.v_page_stride | g.v_slot_stride | g.v_head_stride) & 7)
        return 0;
    // 31-bit key positions, rows and slot byte offsets (the kernel's scalar arithmetic)
    const int64_t lim = (int64_t)1 << 30;
    const int64_t slots = P.bt ? ((int64_t)1 << P.pshift) : (int64_t)g.max_seq_len + 64;
    if (P.rows >= lim || (int64_t)g.max_seq_len + 64 >= lim) return 0;
    if (slots * 2 * g.k_slot_stride >= lim || slots * 2 * g.v_slot_stride >= lim) return 0;
    return 1;
}

namespace {
// page lookups every PGL keys, PGL <= page size (one lookup per 64-key tile without a table)
const void* decode_fn_for(const Params& P, bool stream) {
    const int pgl = !P.bt ? 64 : (P.pshift >= 6 ? 64 : (P.pshift >= 4 ? 16 : 4));
    if (stream) return P.rb == 1 ? decode_fn<1, true>(pgl) : decode_fn<2, true>(pgl);
    return P.rb == 1 ? decode_fn<1, false>(pgl) : decode_fn<2, false>(pgl);
}
size_t decode_lds(int rb) { return rb == 1 ? sizeof(DecodeSmem<1>) : sizeof(DecodeSmem<2>); }
hipError_t decode_attrs() {
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    std::call_once(once, [] {
        const void* fns[12] = {decode_fn<1, false>(4), decode_fn<1, false>(16), decode_fn<1, false>(64),
                               decode_fn<2, false>(4), decode_fn<2, false>(16), decode_fn<2, false>(64),
                               decode_fn<1, true>(4),  decode_fn<1, true>(16),  decode_fn<1, true>(64),
                               decode_fn<2, true>(4),  decode_fn<2, true>(16),  decode_fn<2, true>(64)};
        for (const void* f : fns) {
            hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(DecodeSmem<2>));
            if (e != hipSuccess) attr_err = e;
        }
    });
    return attr_err;
}
}  // namespace

int ea::ea_decode_slots(const Params& P, int* slots, int* cus_out) {
    // blocks of the decode kernel resident on the current device at once (CUs x blocks per CU),
    // and the CU count, cached per device and row-block size
    static std::mutex mu;
    static int cache[64][2] = {};
    static int cache_cus[64][2] = {};
    hipError_t e = decode_attrs();
    if (e != hipSuccess) return -100 - (int)e;
    int dev = 0;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return -100 - (int)e;
    const int ri = P.rb == 1 ? 0 : 1;
    std::lock_guard<std::mutex> lk(mu);
    if (dev < 0 || dev >= 64) return -1;
    if (!cache[dev][ri]) {
        int cus = 0, per = 0;
        if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return -100 - (int)e;
        if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, decode_fn_for(P, true), 128, decode_lds(P.rb))) !=
            hipSuccess)
            return -100 - (int)e;
        cache[dev][ri] = (cus > 0 ? cus : 1) * (per > 0 ? per : 1);
        cache_cus[dev][ri] = cus > 0 ? cus : 1;
    }
    *slots = cache[dev][ri];
    if (cus_out) *cus_out = cache_cus[dev][ri];
    return 0;
}

int ea::ea_launch_decode(const Params& P, hipStream_t st) {
    hipError_t e = decode_attrs();
    if (e != hipSuccess) return -100 - (int)e;
    Params Pc = P;
    void* args[] = {&Pc};
    const dim3 grid = P.dq_stream ? dim3((unsigned)P.dq_blocks) : dim3((unsigned)(P.nseg * P.nrb), (unsigned)P.nsplit);
    e = hipLaunchKernel(decode_fn_for(P, P.dq_stream != 0), grid, dim3(128), args, decode_lds(P.rb), st);
    return e == hipSuccess ? 0 : -100 - (int)e;
}
