// Shared kernel parameters and wave-level helpers of the certified attention kernels (gfx950).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/exactattn_hip.h"
#include "ea_device.h"

namespace ea {

#define EA_TILE 64
#define EA_THREADS 256
#define EA_MAXRB 4
#define EA_MAXD 128
#define EA_MAXDV 128
#define EA_T2_BLOCKS 32

// ------------------------------------------------------------------------------------------------
// Kernel parameters
// ------------------------------------------------------------------------------------------------
struct Params {
    ea_geometry g;
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const int32_t* seq_len;
    const int32_t* kv_len;
    const int32_t* bt;
    const int64_t* bt_off;
    const uint64_t* tree_mask;
    const int32_t* tree_base;
    void* out;
    uint8_t* flags;
    int64_t* stats;
    int64_t* timers;
    const int32_t* merge_order;
    double alpha;
    int32_t am, ae;
    int32_t out_fp32;
    int32_t nsplit, split_len;
    int32_t grp, r_seg, rb, nrb, nseg;
    int32_t pshift;
    int32_t dlog;
    int64_t rows;
    // workspace
    double* q64;      // rows * EA_MAXD
    int32_t* qinfo;   // rows * 5: per 32-dim block (FQmax << 16) | FQmin', then a NaN/inf flag
    double* qn;       // rows * 4: per 32-dim block an upper bound of sum |q_i| (fp64)
    int32_t* pR;      // nsplit * rows
    int32_t* pn;      // nsplit * rows (visible keys, or -1 for a tier-1 flag)
    double* pZ;       // nsplit * rows
    double* pN;       // nsplit * rows * dv
    float* pV;        // nsplit * nseg * nrb * dv : max |v| per channel over the block's keys
    int32_t* wl;      // rows
    int32_t* wl_cnt;  // 1 + EA_T2_BLOCKS: the work list's length, then tier 2's per-row chunk counts
    void* t2part;     // EA_T2_BLOCKS tier-2 chunk partials (T2Part, ea_hip.hip)
    int32_t* t2M;     // EA_T2_BLOCKS * max_keys
    int64_t* t2E;     // EA_T2_BLOCKS * max_keys
    int32_t t2_keys;
    // int8-MFMA prefill path (ea_prefill.hip)
    uint8_t* pfq;     // rows * 512: q digit planes
    void* pfqm;       // rows * sizeof(PfQMeta)
    uint8_t* pfkv;    // nseg * pf_ntiles * EA_PF_TILE_BYTES: K/V digit tiles and tile metadata
    double* pfscr;    // nseg * pf_nrb * 512 lanes * 32: per-lane sums of completed epochs
    int32_t pf_ntiles;  // 64-key tiles per segment
    int32_t pf_nrb;     // 32-row blocks per segment
    // digit-tile cache (ea_hip_kv_digits_update): with kvd_begin set, ea_pf_kvslice re-slices the
    // tiles that hold keys [kvd_begin[b], kvd_end[b]) of each sequence, kvd_span tiles per segment
    const int32_t* kvd_begin;
    const int32_t* kvd_end;
    int32_t kvd_span;
    int32_t pf_kv_cached;  // 1: pfkv is the caller's digit cache, already sliced
    const int32_t* pf_kv_slot;  // with pf_kv_cached: cache slot of each sequence (NULL: b)
    int32_t pf_waves;           // prefill block shape: 8 waves (default) or 4
    int32_t pf_nsplit;          // key splits per (segment, row block); 1: rounding in ea_pf_main
    int32_t pf_tps;             // 64-key tiles per key split
    void* pf_part;              // pf_nsplit > 1: the splits' partials (PfPart, then PfEntry arrays)
    // Equal-share decomposition of the d = 128 decode kernel (dq_stream = 1). The step's 64-key
    // tiles, unit by unit (unit = (segment, row block), tiles up to its visible end), are cut into
    // dq_blocks consecutive shares of `share` tiles; block g takes share g, which is one or more
    // pieces (its intersections with units), and writes piece p of unit u in partial slot p,
    // p = g - floor(S_u / share). dq_plan, written by the prep kernel's planner block: [0] W
    // (tiles), [1] share, [2 + u] S_u for u = 0 .. dq_units (prefix sums, S_units = W), then
    // at dq_rec_off (16-byte aligned) per block g its first piece (u, S_u, S_(u+1), share), u =
    // dq_units for a block past the last tile. share >= dq_min_share keeps every unit within
    // nsplit pieces.
    int32_t dq_stream;
    int32_t dq_units;
    int32_t dq_blocks;
    int32_t dq_min_share;
    int32_t dq_max_tiles;
    int32_t dq_rec_off;
    int32_t* dq_plan;
    // Most 64-key tiles in one partial of the d = 128 decode kernel (split_len / 64, the longest
    // weighted split, or the share of its equal-share plan); 0 when another kernel wrote the
    // partials. The combine's error bound uses it: the kernel's lane chains hold at most 16 keys of
    // each tile.
    int32_t pv_tiles;
    // Uniform decode grid of exactly one round of resident blocks: the first dq_lead blocks in
    // dispatch order (one per CU) run ahead of the rest (about 1.2x), so a unit's key range
    // [0, nsplit split_len) is cut in whole tiles in proportion to weights 5 for its splits among
    // them and 4 for the others. 0: equal splits of split_len.
    int32_t dq_lead;
};

__device__ __forceinline__ int64_t row_index(const Params& P, int64_t b, int t, int hq) {
    return (b * P.g.num_tokens + t) * P.g.num_q_heads + hq;
}

// The key range a decode unit (segment seg, row block rbk of P.rb rows) reads: keys below the
// largest visible end of its rows (prefix kv_len, tree keys tree_base + i), clipped to seq_len.
// The decode kernel and the planner of its equal-share decomposition both use it.
__device__ inline int unit_kend(const Params& P, int seg, int rbk) {
    const int Hkv = P.g.num_kv_heads;
    const int b = seg / Hkv;
    const int row0 = rbk * P.rb;
    const int nrow = min(P.rb, P.r_seg - row0);
    const int tb = P.tree_mask ? P.tree_base[b] : 0;
    int kend = 0;
    for (int r = 0; r < nrow; ++r) {
        const int t = (row0 + r) / P.grp;
        const int64_t tok = (int64_t)b * P.g.num_tokens + t;
        int e = P.kv_len[tok];
        const uint64_t m = P.tree_mask ? P.tree_mask[tok] : 0ull;
        if (m) e = max(e, tb + 64 - (int)__clzll(m));
        kend = max(kend, e);
    }
    return min(kend, (int)P.seq_len[b]);
}

// global element offset of key n of sequence b, kv head hk (K when isv = 0, V when 1)
__device__ __forceinline__ int64_t kv_off(const Params& P, int64_t b, int64_t n, int hk, int isv) {
    int64_t page, slot;
    if (P.bt) {
        int64_t off = P.bt_off ? P.bt_off[b] : b * (int64_t)P.g.block_table_stride;
        page = P.bt[off + (n >> P.pshift)];
        slot = n & ((1 << P.pshift) - 1);
    } else {
        page = b;
        slot = n;
    }
    if (isv) return page * P.g.v_page_stride + slot * P.g.v_slot_stride + (int64_t)hk * P.g.v_head_stride;
    return page * P.g.k_page_stride + slot * P.g.k_slot_stride + (int64_t)hk * P.g.k_head_stride;
}

__device__ __forceinline__ bool visible(const Params& P, int64_t tok, int64_t b, int64_t n) {
    if (n < P.kv_len[tok]) return true;
    if (P.tree_mask) {
        int64_t i = n - P.tree_base[b];
        if (i >= 0 && i < 64) return (P.tree_mask[tok] >> i) & 1;
    }
    return false;
}

// The visible keys of a query token, the set every tier attends: the prefix n < Lc with
// Lc = min(kv_len, seq_len) (0 when kv_len < 0), and the tree keys tree_base + i (bit i of the tree
// mask) at or past Lc and below seq_len, so a key in both counts once. vis_tree_bits keeps those
// tree bits; the prefix clip is the caller's. Host and device.
__host__ __device__ inline uint64_t vis_tree_bits(uint64_t mask, int64_t tb, int64_t Lc, int64_t slen) {
    int64_t lo = Lc - tb, hi = slen - tb;  // keep bits i with lo <= i < hi
    lo = lo < 0 ? 0 : (lo > 64 ? 64 : lo);
    hi = hi < 0 ? 0 : (hi > 64 ? 64 : hi);
    if (hi <= lo) return 0;
    const uint64_t below_hi = hi >= 64 ? ~0ull : ((1ull << hi) - 1);
    const uint64_t below_lo = lo >= 64 ? ~0ull : ((1ull << lo) - 1);
    return mask & below_hi & ~below_lo;
}
__host__ __device__ inline int64_t vis_prefix(int64_t kv_len, int64_t slen) {
    return kv_len < 0 ? 0 : (kv_len < slen ? kv_len : slen);
}

// end of the visible key range of a query token
__device__ __forceinline__ int64_t vis_end(const Params& P, int64_t tok, int64_t b) {
    int64_t e = P.kv_len[tok];
    if (P.tree_mask) {
        uint64_t m = P.tree_mask[tok];
        if (m) {
            int64_t te = P.tree_base[b] + 64 - __clzll(m);
            if (te > e) e = te;
        }
    }
    return e;
}

// Max over the 64 lanes with DPP row shifts and row broadcasts (no LDS round trip); every lane
// receives the result. gfx9 DPP controls: row_shr:n = 0x110 + n, row_bcast:15 = 0x142,
// row_bcast:31 = 0x143; lanes without a source keep their own value (the max identity here).
__device__ __forceinline__ int wave_max_dpp(int x) {
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x111, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x112, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x114, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x118, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x142, 0xA, 0xF, false));
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x143, 0xC, 0xF, false));
    return __builtin_amdgcn_readlane(x, 63);
}

// Max within each 16-lane DPP row (lanes 16r .. 16r+15); every lane of the row receives it.
__device__ __forceinline__ int row16_max(int x) {
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x111, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x112, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x114, 0xF, 0xF, false));
    x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x118, 0xF, 0xF, false));
    // lane 15 of each row now holds the row's max: broadcast it within the row
    return __shfl(x, (threadIdx.x & 48) | 15, 64);
}

__device__ __forceinline__ double wave_sum(double x) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}
__device__ __forceinline__ int wave_max_i(int x) {
    for (int o = 32; o > 0; o >>= 1) x = max(x, __shfl_xor(x, o, 64));
    return x;
}
__device__ __forceinline__ int wave_min_i(int x) {
    for (int o = 32; o > 0; o >>= 1) x = min(x, __shfl_xor(x, o, 64));
    return x;
}
__device__ __forceinline__ int wave_sum_i(int x) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}


// The d = dv = 128 decode kernel (ea_decode.hip). ea_decode_eligible: 1 when P's geometry and
// pointers allow it (else the general split kernel runs). ea_decode_slots: blocks resident on the
// current device at once. ea_launch_decode: P.dq_blocks blocks over the equal-share plan (0 or
// -100 - e on a HIP error).
int ea_decode_eligible(const Params& P);
int ea_decode_slots(const Params& P, int* slots, int* cus = nullptr);
int ea_launch_decode(const Params& P, hipStream_t st);

// int8-MFMA prefill path (ea_prefill.hip). A tile holds 64 keys of one segment:
//   [0, 32768)       K digit planes t = 0..3: [t][key 64][128 bytes], 16-byte chunk c of key k
//                    stored at chunk c ^ (k & 7)
//   [32768, 65536)   V digit planes t = 0..3: [t][channel 128][64 bytes], key 16kt + 4g + i at
//                    byte 16 (g ^ ((channel >> 1) & 3)) + 4kt + i
//   [65536, 69632)   PfTileMeta
#define EA_PF_TILE_BYTES 69632
#define EA_PF_META_OFF 65536
struct PfQMeta {
    int32_t lsb;    // q = X * 2^lsb, |X| < 2^30
    int32_t flags;  // bit 0: digit 0 nonzero somewhere; bit 1: NaN/inf; bits 8..15: inexact elements
    double qA;      // sum_i sum_s |d_s,i| 2^(8s)
    double qX;      // max_i |X_i|
    double a;       // alpha * 2^lsb
};
struct PfTileMeta {
    int32_t lsbk[64];
    int32_t vlsb[64];
    double kA[64];    // max_i sum_t |d_t,i| 2^(8t)
    double kX[64];    // max_i |X_i|
    int32_t kfl[64];  // bit 0: NaN/inf in the key's K or V row; bits 8..15: inexact K elements
    double EV[128];   // per channel: (2^38 + 1) / 2 * (inexact V elements of the tile)
    int32_t tfl;      // bit kt: a key of 16-key group kt needs K digit 0; bit 4: a NaN/inf key;
                      // bit 5: a key with inexact K elements
    int32_t pad;
    double EVt;       // (2^38 + 1) / 2 * (inexact V elements of the tile, all channels)
};
// A key split's partial of one row (pf_nsplit > 1): the row's base exponent, its visible keys with
// a weight, bit 0 a domain error and bit 1 an undecided pair, Z in units 2^base. Followed in the
// workspace by the (N, bound) pairs of every (split, row, channel), also in units 2^base.
struct PfPart {
    int32_t base;
    int32_t nv;
    int32_t fl;
    int32_t pad;
    double z;
    double pad2;
};
// Returns 1 when the prefill path handles this geometry (and sets the tile and block counts),
// 0 otherwise. kernel: the ea_options.kernel choice (EA_KERNEL_*).
int ea_prefill_eligible(const ea_geometry& g, int grp, int kernel, int* ntiles, int* nrb);
// Enqueue the slicing kernels (q rows, K/V tiles), then the prefill kernel; 0 or -100 - e.
int ea_launch_prefill(const Params& P, hipStream_t st);
int ea_launch_prefill_main(const Params& P, hipStream_t st);
// With key splits (P.pf_nsplit > 1): the merge of the splits' partials and the rounding.
int ea_launch_prefill_combine(const Params& P, hipStream_t st);
// Enqueue the re-slicing of the cached digit tiles P.kvd_begin / kvd_end name; 0 or -100 - e.
int ea_launch_kv_digits(const Params& P, hipStream_t st);

typedef const double __attribute__((address_space(4))) cdouble_t;
typedef const int32_t __attribute__((address_space(4))) cint_t;

// q row `row` prepared by one wave from its bf16 elements x[h] = q[2 lane + h] (dims past the head
// dimension passed as +0): the fp64 row, per 32-dim block (lanes 16 blk .. 16 blk + 15, each
// 16-lane group reduces its block) qinfo[row*5 + blk] = (FQmax << 16) | FQmin' over the nonzero
// elements (FQmin' = max(field, 1): a subnormal's lsb is that of field 1), 0x80000000 for an
// all-zero block, and qn[row*4 + blk] = an upper bound of sum |q_i| (the fp64 sum has at most 32
// roundings of relative size 2^-53 in any order, so times 1 + 2^-40 bounds it; NaN/inf propagate),
// and qinfo[row*5 + 4] = the NaN/inf flag, which it also returns (the same in every lane).
// *qn_blk receives the stored bound of the lane's own block (lane >> 4).
__device__ __forceinline__ int prep_row_store(const Params& P, int64_t row, int lane, uint32_t x0, uint32_t x1,
                                              double* qn_blk = nullptr) {
    const int blk = lane >> 4;
    const uint32_t x[2] = {x0, x1};
    int bad = 0, fmax = 0, fmin = 0x1FF;
    double aq = 0.0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int i = 2 * lane + h;
        const double qv = (double)__uint_as_float(x[h] << 16);
        P.q64[row * EA_MAXD + i] = qv;
        aq += fabs(qv);
        const int f = (x[h] >> 7) & 0xFF;
        if (f == 0xFF) bad = 1;
        if (x[h] & 0x7FFF) {
            fmax = max(fmax, f);
            fmin = min(fmin, max(f, 1));
        }
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
        fmax = max(fmax, __shfl_xor(fmax, o, 64));
        fmin = min(fmin, __shfl_xor(fmin, o, 64));
        aq += __shfl_xor(aq, o, 64);
    }
    const double qb = aq * (1.0 + 0x1p-40);
    if ((lane & 15) == 0) {
        P.qinfo[row * 5 + blk] = (fmin == 0x1FF) ? (int32_t)0x80000000 : ((fmax << 16) | fmin);
        P.qn[row * 4 + blk] = qb;
    }
    if (qn_blk) *qn_blk = qb;
    bad = wave_max_i(bad);
    if (lane == 0) P.qinfo[row * 5 + 4] = bad;
    return bad;
}

}  // namespace ea
