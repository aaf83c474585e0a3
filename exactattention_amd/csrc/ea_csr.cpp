// The reference-compatible drop-in ea_attention_hip (the ABI of the reference's ea_attention_cpu,
// csrc/exact_attention_cpu.cpp:585-628): CSR rows over host arrays, computed on the current HIP
// device by the same kernels a serving geometry takes.
//
// A CSR problem gives each row its own key list. Rows whose lists are prefixes of one list (the
// query heads of one KV head, the tokens of a causal prefix, the rows of a decode batch that
// share a sequence) form a family; a family becomes one sequence of the serving geometry whose
// cache is the family's longest list and whose tokens are its rows (visible prefix = the row's
// list length), so its K/V tiles are read once for all of its rows and the launcher's kernel
// choice applies (the d = 128 decode kernel for a few rows per family, the int8 prefill kernel
// for many). The cache is the caller's K/V array viewed as pages of P keys, P the largest power
// of two up to 64 at which every family list is a sequence of whole aligned runs (P = 1, the
// list itself as the block table, for arbitrary lists). Empty rows are +0 with flag 0 without
// device work; rows the device tiers leave at flag 1 are recomputed by the host exact tier.
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "../../include/exactattn_hip.h"
#include "ea_exact.h"

namespace {

constexpr int kMaxHead = 128;     // this build's largest head sizes (d, dv)
constexpr int kMaxDevices = 64;

int hip_rc(hipError_t e) { return e == hipSuccess ? 0 : -100 - (int)e; }

// Families, tokens and the page view of the caller's key arrays.
struct CsrLayout {
    int32_t page = 1;
    int32_t B = 0, T = 0;
    int32_t max_seq_len = 0;
    std::vector<int64_t> tok_row;  // B*T: the CSR row of each token, -1 for padding
    std::vector<int32_t> kv_len;   // B*T
    std::vector<int32_t> seq_len;  // B
    std::vector<int64_t> bt_off;   // B: where sequence b's pages start in bt
    std::vector<int32_t> bt;       // page numbers of every family's list, concatenated
};

// True when list[0, n) consists of whole runs of P consecutive keys, each starting at a multiple
// of P (the last run may be cut short by n).
bool runs_of(const int64_t* list, int64_t n, int64_t P) {
    for (int64_t i = 0; i < n; ++i) {
        if (i % P == 0) {
            if (list[i] % P) return false;
        } else if (list[i] != list[i - 1] + 1) {
            return false;
        }
    }
    return true;
}

void plan_families(int64_t rows, const int64_t* row_ptr, const int64_t* key_idx, CsrLayout* L) {
    // rows by decreasing list length (a family's first row holds its longest list)
    std::vector<int64_t> order;
    order.reserve((size_t)rows);
    for (int64_t r = 0; r < rows; ++r)
        if (row_ptr[r + 1] > row_ptr[r]) order.push_back(r);
    std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) {
        return row_ptr[a + 1] - row_ptr[a] > row_ptr[b + 1] - row_ptr[b];
    });
    struct Family {
        int64_t base;                // row holding the family's longest list
        std::vector<int64_t> rows;   // decreasing length
    };
    std::vector<Family> fam;
    std::unordered_map<int64_t, std::vector<int32_t>> by_first;  // first key -> families
    for (int64_t r : order) {
        const int64_t n = row_ptr[r + 1] - row_ptr[r];
        const int64_t* lr = key_idx + row_ptr[r];
        std::vector<int32_t>& cand = by_first[lr[0]];
        int32_t hit = -1;
        for (size_t c = 0; c < cand.size() && c < 8 && hit < 0; ++c) {
            const int64_t* lb = key_idx + row_ptr[fam[(size_t)cand[c]].base];
            if (memcmp(lr, lb, (size_t)n * sizeof(int64_t)) == 0) hit = cand[c];
        }
        if (hit < 0) {
            hit = (int32_t)fam.size();
            fam.push_back(Family{r, {}});
            cand.push_back(hit);
        }
        fam[(size_t)hit].rows.push_back(r);
    }
    // page size: the largest power of two (<= 64) at which every family list is aligned runs
    int64_t P = 64;
    for (const Family& f : fam) {
        const int64_t n = row_ptr[f.base + 1] - row_ptr[f.base];
        while (P > 1 && !runs_of(key_idx + row_ptr[f.base], n, P)) P >>= 1;
    }
    L->page = (int32_t)P;
    // tokens per sequence: the largest family, halved while padding would exceed a quarter of
    // the rows (a family longer than T is cut into several sequences over the same pages)
    const int64_t real = (int64_t)order.size();
    int64_t T = 1;
    for (const Family& f : fam) T = std::max<int64_t>(T, (int64_t)f.rows.size());
    auto padded = [&](int64_t t) {
        int64_t s = 0;
        for (const Family& f : fam) s += ((int64_t)f.rows.size() + t - 1) / t * t;
        return s;
    };
    while (T > 1 && padded(T) > real + real / 4 + 64) T = (T + 1) / 2;
    L->T = (int32_t)T;
    int64_t B = 0;
    for (const Family& f : fam) B += ((int64_t)f.rows.size() + T - 1) / T;
    L->B = (int32_t)B;
    L->tok_row.assign((size_t)(B * T), -1);
    L->kv_len.assign((size_t)(B * T), 0);
    L->seq_len.assign((size_t)B, 0);
    L->bt_off.assign((size_t)B, 0);
    L->bt.clear();
    L->max_seq_len = 0;
    int64_t b = 0;
    for (const Family& f : fam) {
        const int64_t n = row_ptr[f.base + 1] - row_ptr[f.base];
        const int64_t* lb = key_idx + row_ptr[f.base];
        const int64_t off = (int64_t)L->bt.size();
        for (int64_t i = 0; i < n; i += P) L->bt.push_back((int32_t)(lb[i] / P));
        // rows in increasing length: a sequence's row blocks hold similar prefixes
        const int64_t m = (int64_t)f.rows.size();
        for (int64_t c0 = 0; c0 < m; c0 += T, ++b) {
            int32_t longest = 0;
            for (int64_t t = 0; t < T && c0 + t < m; ++t) {
                const int64_t r = f.rows[(size_t)(m - 1 - (c0 + t))];
                const int32_t len = (int32_t)(row_ptr[r + 1] - row_ptr[r]);
                L->tok_row[(size_t)(b * T + t)] = r;
                L->kv_len[(size_t)(b * T + t)] = len;
                longest = std::max(longest, len);
            }
            L->seq_len[(size_t)b] = longest;
            L->bt_off[(size_t)b] = off;
            L->max_seq_len = std::max(L->max_seq_len, longest);
        }
    }
}

// One device arena and stream per device, grown as calls need: repeated calls allocate nothing.
// The drop-in is synchronous, so its calls on one device are serialised by the device's lock.
struct Arena {
    std::mutex mu;
    void* base = nullptr;
    size_t cap = 0;
    hipStream_t stream = nullptr;
};
Arena g_arena[kMaxDevices];

size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

int attention_csr(const uint16_t* q, int64_t rows, int d, const uint16_t* k, const uint16_t* v, int64_t nkeys, int dv,
                  float alpha, const int64_t* row_ptr, const int64_t* key_idx, int fp32_out, int acc_bits, int tile,
                  int splits, void* out, uint8_t* flags, int64_t* stats) {
    // the reference's argument checks, in its order (csrc/exact_attention_cpu.cpp:589-592)
    if (d <= 0 || d > kMaxHead || dv <= 0 || dv > kMaxHead || tile <= 0 || splits <= 0) return -1;
    if (acc_bits != 64 && acc_bits != 128) return -2;
    uint32_t alpha_bits;
    memcpy(&alpha_bits, &alpha, 4);
    if (((alpha_bits >> 23) & 0xFF) == 0xFF) return -3;
    if ((d & 7) || (dv & 1) || rows < 0 || nkeys < 0) return -1;
    if (rows == 0) return 0;
    if (rows > INT32_MAX / 2) return -1;  // sequences and tokens of the geometry are int32
    if (!q || !row_ptr || !out || !flags || (nkeys > 0 && (!k || !v))) return -1;
    if (row_ptr[0] < 0) return -1;
    int64_t maxn = 0;
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t len = row_ptr[r + 1] - row_ptr[r];
        if (len < 0) return -1;
        maxn = std::max(maxn, len);
    }
    const int64_t nnz = row_ptr[rows] - row_ptr[0];
    if (maxn > INT32_MAX / 2 || nkeys > INT32_MAX / 2) return -1;
    if (nnz > 0 && !key_idx) return -1;
    for (int64_t j = row_ptr[0]; j < row_ptr[rows]; ++j)
        if (key_idx[j] < 0 || key_idx[j] >= nkeys) return -1;  // the kernels gather through it
    const size_t osz = fp32_out ? 4 : 2;
    // empty rows: +0, certified (the empty set's output)
    for (int64_t r = 0; r < rows; ++r)
        if (row_ptr[r + 1] == row_ptr[r]) {
            memset((char*)out + (size_t)r * dv * osz, 0, (size_t)dv * osz);
            flags[r] = 0;
        }
    if (nnz == 0) return 0;

    CsrLayout L;
    plan_families(rows, row_ptr, key_idx, &L);
    const int64_t P = L.page, BT = (int64_t)L.B * L.T;
    const int64_t npages = (nkeys + P - 1) / P;
    ea_geometry g;
    memset(&g, 0, sizeof(g));
    g.num_seqs = L.B; g.num_tokens = L.T; g.num_q_heads = 1; g.num_kv_heads = 1;
    g.head_dim = d; g.head_dim_v = dv;
    g.q_seq_stride = (int64_t)L.T * d; g.q_tok_stride = d; g.q_head_stride = 0;
    g.o_seq_stride = (int64_t)L.T * dv; g.o_tok_stride = dv; g.o_head_stride = 0;
    g.k_page_stride = P * d; g.k_slot_stride = d; g.k_head_stride = 0;
    g.v_page_stride = P * dv; g.v_slot_stride = dv; g.v_head_stride = 0;
    g.page_size = (int32_t)P; g.block_table_stride = 0; g.max_seq_len = L.max_seq_len;
    ea_options o;
    memset(&o, 0, sizeof(o));
    o.alpha_bits = alpha_bits; o.out_fp32 = fp32_out ? 1 : 0; o.splits = splits; o.tier2 = 1;
    size_t ws_bytes = 0;
    int32_t ns = 0;
    int rc = ea_hip_workspace_size(&g, &o, &ws_bytes, &ns);
    if (rc) return rc;

    // q rows in token order (padding tokens zero), and the host side of the results: every host
    // buffer a copy reads or writes exists before the first copy is enqueued
    std::vector<uint16_t> qh((size_t)(BT * d), 0);
    for (int64_t i = 0; i < BT; ++i)
        if (L.tok_row[(size_t)i] >= 0) memcpy(&qh[(size_t)(i * d)], q + L.tok_row[(size_t)i] * d, (size_t)d * 2);
    std::vector<unsigned char> oh((size_t)BT * dv * osz);
    std::vector<uint8_t> fh((size_t)BT);
    int64_t hs[16] = {};

    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_rc(e);
    if (dev < 0 || dev >= kMaxDevices) return -1;
    Arena& A = g_arena[dev];
    std::lock_guard<std::mutex> lk(A.mu);
    if (!A.stream && (e = hipStreamCreateWithFlags(&A.stream, hipStreamNonBlocking)) != hipSuccess) return hip_rc(e);
    // arena layout
    const size_t kv_rows = (size_t)(npages * P);
    size_t off = 0;
    const size_t o_q = off; off = up256(off + (size_t)BT * d * 2);
    const size_t o_k = off; off = up256(off + kv_rows * d * 2);
    const size_t o_v = off; off = up256(off + kv_rows * dv * 2);
    const size_t o_bt = off; off = up256(off + L.bt.size() * 4);
    const size_t o_bo = off; off = up256(off + (size_t)L.B * 8);
    const size_t o_sl = off; off = up256(off + (size_t)L.B * 4);
    const size_t o_kl = off; off = up256(off + (size_t)BT * 4);
    const size_t o_out = off; off = up256(off + (size_t)BT * dv * osz);
    const size_t o_fl = off; off = up256(off + (size_t)BT);
    const size_t o_st = off; off = up256(off + 16 * sizeof(int64_t));
    const size_t o_ws = off; off = up256(off + std::max<size_t>(ws_bytes, 256));
    if (off > A.cap) {
        if (A.base) (void)hipFree(A.base);
        A.base = nullptr;
        A.cap = 0;
        if ((e = hipMalloc(&A.base, off)) != hipSuccess) return hip_rc(e);
        A.cap = off;
    }
    char* base = (char*)A.base;
    const hipStream_t st = A.stream;
    // every way out after this point, an error or an exception included, first waits for the
    // stream: no copy may still read or write a host buffer of this call, and no work may still use
    // the arena when a later call regrows it
    struct SyncOnExit {
        hipStream_t s;
        bool armed;
        ~SyncOnExit() {
            if (armed) (void)hipStreamSynchronize(s);
        }
    } guard{st, true};
#define EA_TRY(x)                            \
    do {                                     \
        if ((e = (x)) != hipSuccess) return hip_rc(e); \
    } while (0)
    EA_TRY(hipMemcpyAsync(base + o_q, qh.data(), (size_t)BT * d * 2, hipMemcpyHostToDevice, st));
    EA_TRY(hipMemcpyAsync(base + o_k, k, (size_t)nkeys * d * 2, hipMemcpyHostToDevice, st));
    EA_TRY(hipMemcpyAsync(base + o_v, v, (size_t)nkeys * dv * 2, hipMemcpyHostToDevice, st));
    if (kv_rows > (size_t)nkeys) {  // the last page's keys past the array: never read, kept finite
        EA_TRY(hipMemsetAsync(base + o_k + (size_t)nkeys * d * 2, 0, (kv_rows - (size_t)nkeys) * d * 2, st));
        EA_TRY(hipMemsetAsync(base + o_v + (size_t)nkeys * dv * 2, 0, (kv_rows - (size_t)nkeys) * dv * 2, st));
    }
    EA_TRY(hipMemcpyAsync(base + o_bt, L.bt.data(), L.bt.size() * 4, hipMemcpyHostToDevice, st));
    EA_TRY(hipMemcpyAsync(base + o_bo, L.bt_off.data(), (size_t)L.B * 8, hipMemcpyHostToDevice, st));
    EA_TRY(hipMemcpyAsync(base + o_sl, L.seq_len.data(), (size_t)L.B * 4, hipMemcpyHostToDevice, st));
    EA_TRY(hipMemcpyAsync(base + o_kl, L.kv_len.data(), (size_t)BT * 4, hipMemcpyHostToDevice, st));
    EA_TRY(hipMemsetAsync(base + o_st, 0, 16 * sizeof(int64_t), st));
    ea_buffers bf;
    memset(&bf, 0, sizeof(bf));
    bf.q = (const uint16_t*)(base + o_q);
    bf.k = (const uint16_t*)(base + o_k);
    bf.v = (const uint16_t*)(base + o_v);
    bf.seq_len = (const int32_t*)(base + o_sl);
    bf.kv_len = (const int32_t*)(base + o_kl);
    bf.block_table = (const int32_t*)(base + o_bt);
    bf.block_table_offset = (const int64_t*)(base + o_bo);
    bf.out = base + o_out;
    bf.flags = (uint8_t*)(base + o_fl);
    o.stats = (int64_t*)(base + o_st);
    if ((rc = ea_hip_attention(&g, &bf, &o, base + o_ws, ws_bytes, (ea_stream_t)st))) return rc;
    EA_TRY(hipMemcpyAsync(oh.data(), base + o_out, oh.size(), hipMemcpyDeviceToHost, st));
    EA_TRY(hipMemcpyAsync(fh.data(), base + o_fl, fh.size(), hipMemcpyDeviceToHost, st));
    EA_TRY(hipMemcpyAsync(hs, base + o_st, sizeof(hs), hipMemcpyDeviceToHost, st));
    guard.armed = false;
    EA_TRY(hipStreamSynchronize(st));
#undef EA_TRY
    for (int64_t i = 0; i < BT; ++i) {
        const int64_t r = L.tok_row[(size_t)i];
        if (r < 0) continue;
        memcpy((char*)out + (size_t)r * dv * osz, &oh[(size_t)i * dv * osz], (size_t)dv * osz);
        flags[r] = fh[(size_t)i];
    }
    if (stats) {
        stats[0] += hs[5];
        stats[1] += hs[6];
        stats[2] += hs[7];
    }
    // rows the device tiers left uncertified: the host exact tier on the caller's arrays
    std::vector<uint16_t> kr, vr;
    for (int64_t r = 0; r < rows; ++r) {
        if (flags[r] != 1) continue;
        const int64_t j0 = row_ptr[r], n = row_ptr[r + 1] - row_ptr[r];
        kr.resize((size_t)(n * d));
        vr.resize((size_t)(n * dv));
        for (int64_t j = 0; j < n; ++j) {
            memcpy(&kr[(size_t)(j * d)], k + key_idx[j0 + j] * d, (size_t)d * 2);
            memcpy(&vr[(size_t)(j * dv)], v + key_idx[j0 + j] * dv, (size_t)dv * 2);
        }
        char* dst_row = (char*)out + (size_t)r * dv * osz;
        const int x = eax::exact_row(q + r * d, d, kr.data(), vr.data(), n, dv, alpha_bits, fp32_out ? 1 : 0, dst_row,
                                     nullptr);
        if (x == eax::EAX_NOMEM) return EA_ERR_HOST_MEMORY;
        if (x != eax::EAX_OK) memset(dst_row, 0, (size_t)dv * osz);
        flags[r] = x == eax::EAX_OK ? 0 : 2;
    }
    return 0;
}

}  // namespace

extern "C" int ea_attention_hip(const uint16_t* q, int64_t rows, int d, const uint16_t* k, const uint16_t* v,
                                int64_t nkeys, int dv, float alpha, const int64_t* row_ptr, const int64_t* key_idx,
                                int fp32_out, int acc_bits, int tile, int splits, uint64_t order_seed, int nthreads,
                                void* out, uint8_t* flags, int64_t* stats) {
    (void)order_seed;
    (void)nthreads;
    try {
        return attention_csr(q, rows, d, k, v, nkeys, dv, alpha, row_ptr, key_idx, fp32_out, acc_bits, tile, splits,
                             out, flags, stats);
    } catch (...) {  // host vectors and maps: only an exhausted heap throws
        return EA_ERR_HOST_MEMORY;
    }
}

// The layout the drop-in gives a CSR problem, for callers that build the same geometry themselves
// (the Python CSR path) and for tests. dims[0..5] = sequences B, tokens per sequence T, page size,
// longest list, block-table entries, B*T. With the array pointers set, also the token -> row map
// (-1 for padding), the visible lengths, sequence lengths, block-table offsets and entries. Host
// only; no device call.
extern "C" int ea_csr_layout(int64_t rows, const int64_t* row_ptr, const int64_t* key_idx, int64_t nkeys, int64_t* dims,
                             int64_t* tok_row, int32_t* kv_len, int32_t* seq_len, int64_t* bt_off, int32_t* bt) {
    if (rows < 0 || !row_ptr || !dims) return -1;
    if (rows > INT32_MAX / 2 || nkeys < 0 || nkeys > INT32_MAX / 2) return -1;
    try {
        if (rows > 0 && row_ptr[0] < 0) return -1;
        for (int64_t r = 0; r < rows; ++r)
            if (row_ptr[r + 1] < row_ptr[r]) return -1;
        if (rows > 0 && row_ptr[rows] > row_ptr[0] && !key_idx) return -1;
        for (int64_t j = rows > 0 ? row_ptr[0] : 0; rows > 0 && j < row_ptr[rows]; ++j)
            if (key_idx[j] < 0 || key_idx[j] >= nkeys) return -1;
        CsrLayout L;
        plan_families(rows, row_ptr, key_idx, &L);
        const int64_t BT = (int64_t)L.B * L.T;
        dims[0] = L.B;
        dims[1] = L.T;
        dims[2] = L.page;
        dims[3] = L.max_seq_len;
        dims[4] = (int64_t)L.bt.size();
        dims[5] = BT;
        if (tok_row) memcpy(tok_row, L.tok_row.data(), (size_t)BT * 8);
        if (kv_len) memcpy(kv_len, L.kv_len.data(), (size_t)BT * 4);
        if (seq_len) memcpy(seq_len, L.seq_len.data(), (size_t)L.B * 4);
        if (bt_off) memcpy(bt_off, L.bt_off.data(), (size_t)L.B * 8);
        if (bt) memcpy(bt, L.bt.data(), L.bt.size() * 4);
        return 0;
    } catch (...) {
        return EA_ERR_HOST_MEMORY;
    }
}
