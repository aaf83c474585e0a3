/*
 * exactattn_hip: certified split-KV ExactAttention on AMD Instinct MI355X (gfx950).
 *
 * C ABI of libexactattn_hip.so. Plain pointers, sizes and a hipStream_t; no torch types.
 * Every returned bf16/fp32 bit pattern equals the ExactAttention definition (the reference's
 * docs/SPEC.md): o_c = RN(N_c / Z) with exact scores, t = RN32(alpha*s), w = RN24(2^t).
 *
 * Return codes: 0 = success; -1 invalid shape/geometry, -2 invalid option, -3 non-finite alpha
 * (the same convention as the reference's ea_attention_cpu, csrc/exact_attention_cpu.cpp:589-592);
 * -5 when the host heap is exhausted (host exact tier and drop-in only); -100 - e for a HIP
 * runtime error e. Nothing throws across this ABI: every entry point catches on its side.
 *
 * Per-row flags (uint8), the reference's meaning (csrc/exact_attention_cpu.cpp:580-584):
 *   0 = certified (bits equal the definition)
 *   1 = not certified by the device tiers (the row's output is +0 and must not be used):
 *       ea_hip_exact_rows recomputes such rows exactly on the host and clears the flag
 *   2 = domain error: a NaN/inf input in the row's visible set, or an fp32 logit overflow (and,
 *       from the host exact tier only, a row whose rounding would need exact sums over an
 *       exponent spread above 2^20 bits, where the reference raises its domain error too,
 *       src/exactattn/reference.py:27-30,124-125)
 */
#ifndef EXACTATTN_HIP_H
#define EXACTATTN_HIP_H

#include <stddef.h>
#include <stdint.h>

/* Return code of the host-side entry points when the host heap is exhausted. */
#define EA_ERR_HOST_MEMORY (-5)

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* ea_stream_t; /* = hipStream_t */

/*
 * Serving geometry. Rows are (sequence b, token t, query head h), enumerated in that order
 * (flags and stats index them so). Sequence b's keys 0 .. seq_len[b]-1 live in a paged or
 * contiguous cache; query head h reads KV head h / (num_q_heads / num_kv_heads) (GQA).
 *
 * Element addresses, in uint16 elements:
 *   q[b, t, h, i]     = q + b*q_seq_stride + t*q_tok_stride + h*q_head_stride + i
 *   out[b, t, h, c]   = out + b*o_seq_stride + t*o_tok_stride + h*o_head_stride + c (bf16 or fp32 units)
 *   key n of seq b:   page = block_table ? block_table[off_b + n / page_size] : b,
 *                     slot = block_table ? n % page_size : n,
 *                     off_b = block_table_offset ? block_table_offset[b] : b*block_table_stride
 *   K[b, n, hk, i]    = k + page*k_page_stride + slot*k_slot_stride + hk*k_head_stride + i  (V alike)
 * Row (b, t, h) attends keys n < kv_len[b*T + t], plus, with tree_mask, keys tree_base[b] + i for
 * every set bit i of tree_mask[b*T + t] (speculative tree verification); only keys below
 * seq_len[b] count, and a key in both parts counts once (every tier attends this same set).
 * Causal prefill, chunked prefill, decode and verification chains are all kv_len prefixes.
 */
typedef struct ea_geometry {
    int32_t num_seqs, num_tokens, num_q_heads, num_kv_heads, head_dim, head_dim_v;
    int64_t q_seq_stride, q_tok_stride, q_head_stride;
    int64_t o_seq_stride, o_tok_stride, o_head_stride;
    int64_t k_page_stride, k_slot_stride, k_head_stride;
    int64_t v_page_stride, v_slot_stride, v_head_stride;
    int32_t page_size;          /* power of two; ignored without a block table */
    int32_t block_table_stride; /* entries per sequence when block_table_offset is NULL */
    int32_t max_seq_len;        /* >= every seq_len[b] (sizes the split grid) */
    int32_t pad0;
} ea_geometry;

/* Device pointers. seq_len, kv_len required; block_table, block_table_offset, tree_mask,
 * tree_base optional (NULL). out: bf16 bits (uint16) or fp32; flags: one uint8 per row. */
typedef struct ea_buffers {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const int32_t* seq_len;
    const int32_t* kv_len;
    const int32_t* block_table;
    const int64_t* block_table_offset;
    const uint64_t* tree_mask;
    const int32_t* tree_base;
    void* out;
    uint8_t* flags;
} ea_buffers;

typedef struct ea_options {
    uint32_t alpha_bits;    /* fp32 bit pattern of the base-2 logit scale */
    int32_t out_fp32;       /* 0 = bf16 output, 1 = fp32 output */
    int32_t splits;         /* KV splits per segment; 0 = choose for the device */
    int32_t tier2;          /* 1 = run the device tier 2 on rows tier 1 leaves uncertified */
    const int32_t* merge_order; /* optional device permutation of [0, nsplit): combine order */
    int64_t* stats;         /* optional device int64[16], accumulated (+=):
                               [0] rows, [1] rows flagged by tier 1, [2] rows certified by tier 2,
                               [3] rows left flag 1, [4] rows flag 2, [5] tier-1 scores not
                               certified, [6] tier-1 weights not certified, [7] tier-1 final
                               roundings not certified, [8] scores taken by the per-pair exact
                               path, [9] rows whose tier 1 ran in the d = 128 decode
                               kernel, [10] rows whose tier 1 ran in the int8-MFMA
                               prefill kernel, [11] prefill epoch folds before the last
                               tile (waves), [12] prefill waves that ran the exact
                               per-pair path, [13] rows certified by the host exact
                               tier (ea_hip_exact_rows), [14] rows it refused (spread
                               limit, flag 2), [15] steps whose decode kernel ran
                               the equal-share plan */
    void* const* events;    /* optional: 5 hipEvent_t recorded on `stream` before prep (the
                               int8 path: q and K/V slicing; none on the decode kernel's uniform
                               grid, whose kernel converts q), the tier-1 kernel, the combine (the
                               int8 path: the merge of its key splits, when it has any) and tier 2,
                               and after tier 2 (per-kernel timing); a null entry is skipped (each
                               record is one more packet in the stream) */
    int64_t* timers;        /* optional device int64[16]: when set, the split kernel runs its
                               phase-clock build and adds shader-clock cycles (s_memtime) summed
                               over waves: [0] prologue, [1] wait for the tile barrier, [2] scores,
                               [3] wait for the score barrier, [4] logits and weights, [5] P.V,
                               [6] epilogue, [7] tiles; the reference's TIMERS build
                               (src/exactattn/triton_kernels.py:747-766) */
    void* kv_digits;        /* optional: the caller's int8 digit-tile cache of K/V
                               (ea_hip_kv_digits_update). When set and the step takes the int8
                               prefill path, its K/V tiles are read there and nothing is sliced;
                               the other paths read the bf16 cache and ignore it */
    int32_t kv_digits_tiles; /* tiles per (sequence, KV head) in kv_digits; must be at least
                               ceil(max_seq_len / 64) */
    int32_t pad1;
    const int32_t* kv_digits_slot; /* optional, with kv_digits: device array, per sequence b of
                               the geometry the cache slot holding its tiles (a serving loop's
                               sequence slot); NULL: slot b */
    int32_t force_tier2;    /* 1: list every row for the device tier 2, whatever tier 1 decided
                               (tier 2 then recomputes and rewrites every row: a test of the
                               exact tier on whole problems; needs tier2 = 1) */
    int32_t kernel;         /* tier-1 kernel: EA_KERNEL_AUTO (by geometry), EA_KERNEL_PREFILL (the
                               int8 prefill kernel for every d = dv = 128 problem),
                               EA_KERNEL_DECODE (never the prefill kernel), EA_KERNEL_GENERAL (the
                               general fp64 split kernel for every problem); never changes bits */
    int32_t prefill_waves;  /* prefill block shape: 0 or 8 = 8 waves, 4 = 4 waves (same bits) */
    int32_t pad2;
} ea_options;

#define EA_KERNEL_AUTO 0
#define EA_KERNEL_PREFILL 1
#define EA_KERNEL_DECODE 2
#define EA_KERNEL_GENERAL 3

/* Bytes of device workspace ea_hip_attention needs for this geometry and options. Also reports
 * the split count it will use: the KV splits per (sequence, KV head), given or chosen; the d = 128
 * decode kernel reads the same count as a bound and divides the step's key tiles into equal shares
 * across the grid (at most nsplit + 1 pieces per segment and row block). Reference counterpart:
 * none (the Triton launcher allocates its partial buffers itself,
 * src/exactattn/triton_kernels.py:1411-1448). */
int ea_hip_workspace_size(const ea_geometry* g, const ea_options* o, size_t* bytes, int32_t* nsplit);

/* Whether ea_hip_attention with this geometry and these options reads o->kv_digits: *reads = 1
 * when kv_digits is set and the step takes the int8 prefill path, else 0. A caller that re-slices
 * its digit-tile cache lazily (only the tiles appends made stale, and only when they are read)
 * brings the cache up to date before exactly these calls. Returns 0 or the negative codes of
 * ea_hip_workspace_size. Reference counterpart: none (the reference slices the whole cache at
 * every launch, src/exactattn/triton_kernels.py:1255-1280). */
int ea_hip_reads_kv_digits(const ea_geometry* g, const ea_options* o, int32_t* reads);

/* Enqueue one certified attention step on `stream`: q prep (inside the tier-1 kernel on the d =
 * 128 decode kernel's uniform grid), tier-1 split kernel, combine with
 * certified rounding, device tier 2 for rows tier 1 could not certify. No host transfer, no
 * synchronisation, fixed grids: capturable in a hipGraph. The caller owns every buffer; the
 * library retains nothing after the work completes.
 * Replaces launch() of src/exactattn/triton_kernels.py:1324-1519 (split kernel + combine +
 * tier 2), extended with paged KV, GQA segments and tree masks. Returns 0; -1 for a bad geometry
 * or a missing buffer, -2 for bad options or a workspace below ea_hip_workspace_size, -3 for a
 * non-finite alpha, -100 - e on a HIP error. A batch with no rows (num_seqs 0) enqueues nothing
 * and returns 0 after the geometry, option and alpha checks, with no buffer or workspace needed. */
int ea_hip_attention(const ea_geometry* g, const ea_buffers* b, const ea_options* o, void* workspace,
                     size_t workspace_bytes, ea_stream_t stream);

/* ea_hip_attention without a caller workspace, for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The workspace is a fixed array of EA_NOALLOC_SCRATCH_BYTES in device memory that each
 * GPU the library runs on holds until the process ends; the call allocates nothing. Geometries
 * whose ea_hip_workspace_size exceeds it return -4 (decode and verification steps fit: C2 needs
 * about 5 MB, long-context decode of 16 sequences up to 131,072 keys about 72 MB; int8 prefill
 * steps of many tokens do not). Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (two streams, two threads) race and must be serialised by the caller. The first call
 * on each device resolves the array's device address (hipGetSymbolAddress): make it outside
 * stream capture; later calls may be captured. Same buffers, options, return codes and stream
 * semantics as ea_hip_attention otherwise (enqueue only, no sync). */
#define EA_NOALLOC_SCRATCH_BYTES (128u << 20)
int ea_hip_attention_noalloc(const ea_geometry* g, const ea_buffers* b, const ea_options* o, ea_stream_t stream);

/* Host exact tier (tier 3) for a step ea_hip_attention enqueued with the same geometry, buffers
 * and options: synchronises `stream`, reads the flags, and recomputes every row left at flag 1
 * exactly on the host (its q, K and V rows gathered on the device into a staging buffer this call
 * allocates and frees), writing the row's bits and flag 0 (flag 2 on a domain error or a refusal,
 * see the flags above). Adds the rows to stats[13] / stats[14] when o->stats is set. Returns 0,
 * -1 on bad arguments, -5 when the host heap is exhausted, -100 - e on a HIP error. Not capturable (it waits for the device).
 * Reference counterpart: the host recompute of flagged rows, src/exactattn/triton_kernels.py:
 * 1553-1559 and src/exactattn/cpu.py:105-108 (reference.attention_row). */
int ea_hip_exact_rows(const ea_geometry* g, const ea_buffers* b, const ea_options* o, ea_stream_t stream);

/* The host exact tier on one row of host arrays: q (d), k (n x d), v (n x dv) bf16 bits, alpha as
 * fp32 bits -> out (dv bf16 or fp32 bits). t_bits, w_m, w_e (optional, n entries each) receive
 * the per-key logits t = RN32(alpha s) and weights w = RN24(2^t) = w_m 2^w_e. Returns 0, 2 for a
 * domain error (NaN/inf input, fp32 logit overflow), 3 when the row needs exact sums over an
 * exponent spread above 2^20 bits, -1 on bad arguments, -5 when the host heap is exhausted.
 * Runs on the CPU only (no device call).
 * Reference counterpart: reference.trace_row / attention_row (src/exactattn/reference.py:82-147). */
int ea_exact_row(const uint16_t* q, int d, const uint16_t* k, const uint16_t* v, int64_t n, int dv,
                 uint32_t alpha_bits, int fp32_out, void* out, uint32_t* t_bits, int32_t* w_m, int64_t* w_e);

/* Drop-in for the reference CPU ABI (csrc/exact_attention_cpu.cpp:585-588): the same argument
 * list, types and return codes as ea_attention_cpu, host pointers; computes on the current HIP
 * device and returns when done. rc -1 for d or dv outside [1, 128] (this build's head sizes;
 * d a multiple of 8, dv even), tile <= 0 or splits <= 0; -2 for acc_bits other than 64 and 128;
 * -3 for a non-finite alpha; -5 when the host heap is exhausted; -100 - e for a HIP error.
 * `tile`, `acc_bits`, `order_seed` and
 * `nthreads` are validated and otherwise ignored (they cannot change certified bits); `splits` is
 * the KV split count. stats[0..2] += tier-1 score, weight and final-rounding fallbacks, as in the
 * reference. Rows the device tiers leave uncertified are recomputed exactly by the host exact
 * tier, so flags are 0, or 2 for rows that see a NaN/inf (their output is +0).
 * Rows whose key lists are prefixes of one list form one sequence of a serving geometry (its
 * cache the caller's K/V viewed as pages of the largest power-of-two run length up to 64 that
 * every list keeps aligned), so the decode and int8 prefill kernels take them and read each
 * shared key once (ea_csr_layout reports the grouping). Device buffers come from a per-device
 * arena kept across calls, on a library stream; calls on one device are serialised. */
int ea_attention_hip(const uint16_t* q, int64_t rows, int d, const uint16_t* k, const uint16_t* v, int64_t nkeys,
                     int dv, float alpha, const int64_t* row_ptr, const int64_t* key_idx, int fp32_out,
                     int acc_bits, int tile, int splits, uint64_t order_seed, int nthreads, void* out,
                     uint8_t* flags, int64_t* stats);

/* The geometry ea_attention_hip gives a CSR problem (rows with no key are not in it: they are +0).
 * dims[0..5] = sequences B (key-list families, each cut to at most T rows), tokens per sequence T,
 * page size P, longest list, block-table entries, B*T. With the optional arrays set, also per
 * token the CSR row (-1 for padding) and visible length, per sequence its length and block-table
 * offset, and the block table (page n holds keys n*P .. n*P + P - 1 of the caller's arrays).
 * Host only. Returns 0, -1 on bad arguments, -5 when the host heap is exhausted. No reference
 * counterpart. */
int ea_csr_layout(int64_t rows, const int64_t* row_ptr, const int64_t* key_idx, int64_t nkeys, int64_t* dims,
                  int64_t* tok_row, int32_t* kv_len, int32_t* seq_len, int64_t* bt_off, int32_t* bt);

/* The reference's test hook (csrc/exact_attention_cpu.cpp:630-638), same signature and result:
 * RN-even of (a / b) * 2^E, a and b as 128-bit (hi, lo) halves, into fp32 (fp32 = 1) or bf16,
 * returned as a float (negated when neg); *overflow = 1 (result 0) when it exceeds the format's
 * largest finite value. Host code only. */
float ea_round_ratio(uint64_t a_hi, uint64_t a_lo, uint64_t b_hi, uint64_t b_lo, int E, int neg, int fp32,
                     int* overflow);

/* Known-answer entry points over the device helper routines (device arrays, n elements).
 * ea_hip_kat_weight: w = RN24(2^t) for fp32 t bits -> M, E, status (0 certified by the fp64
 *   tier-1 path, 1 undecided there; wide tier-2 value in M2/E2 with status2 0/1).
 *   Reference counterpart: exp2.exp2_weight_int_np (src/exactattn/exp2.py:187-195).
 * ea_hip_kat_round: RN of the fp64 interval [x - r, x + r] into bf16/fp32 -> bits, certified.
 *   Reference counterpart: the combine's _ratio_round (src/exactattn/triton_kernels.py:150-195).
 * ea_hip_kat_round_ratio: RN-even of (a/b)*2^E, a,b 128-bit -> bits, overflow.
 *   Reference counterpart: ea_round_ratio (csrc/exact_attention_cpu.cpp:632-638).
 * ea_hip_kat_certify_quotient: tier 2's certified final rounding of N / Z 2^sh over N in
 *   [Nlo, Nhi], Z in [Zlo, Zhi]; `cases` holds 9 int64 per case: Nlo, Nhi, Zlo, Zhi as signed
 *   128-bit (hi, lo) word pairs, then sh -> bits, ok (1 certified). Reference counterpart: the
 *   interval rounding of finalize (csrc/exact_attention_cpu.cpp:450-490). */
int ea_hip_kat_weight(int64_t n, const uint32_t* t_bits, int32_t* M, int64_t* E, int32_t* status, int32_t* M2,
                      int64_t* E2, int32_t* status2, ea_stream_t stream);
int ea_hip_kat_round(int64_t n, const double* x, const double* r, int32_t fp32, uint32_t* bits, int32_t* ok,
                     ea_stream_t stream);
/* ea_hip_kat_wave_max: each 64-lane wave's max of in[64 w .. 64 w + 63] into every lane of out
 * (the DPP reduction the split kernel uses for row maxima and flags). No reference counterpart:
 * the reference's reductions are Triton's tl.max. */
int ea_hip_kat_wave_max(int64_t nwaves, const int32_t* in, int32_t* out, ea_stream_t stream);
int ea_hip_kat_round_ratio(int64_t n, const uint64_t* a_hi, const uint64_t* a_lo, const uint64_t* b_hi,
                           const uint64_t* b_lo, const int32_t* E, const int32_t* neg, int32_t fp32, uint32_t* bits,
                           int32_t* overflow, ea_stream_t stream);
int ea_hip_kat_certify_quotient(int64_t n, const int64_t* cases, int32_t fp32, uint32_t* bits, int32_t* ok,
                                ea_stream_t stream);
/* ea_hip_kat_rn32_prod: the exact logit RN32(am * X * 2^E), X a signed 128-bit integer given as
 * (x_hi signed, x_lo) words, |am| < 2^24 -> fp32 bits, status (0 ok, 2 overflow). The prefill
 * kernel's cold path and tier 2 round exact scores with it.
 * Reference counterpart: certified_logit's exact rounding (csrc/exact_attention_cpu.cpp:215) and
 * RN_fp32(alpha * s) (src/exactattn/reference.py:74-79). */
int ea_hip_kat_rn32_prod(int64_t n, const int32_t* am, const int64_t* x_hi, const uint64_t* x_lo, const int32_t* E,
                         uint32_t* bits, int32_t* status, ea_stream_t stream);

/* The KV slice format as a cache (the write path of a serving loop). For every sequence b and KV
 * head hk, tiles_per_seq tiles of 64 keys, EA_PF_TILE_BYTES = 69632 bytes each, tile t at byte
 * ((b * num_kv_heads + hk) * tiles_per_seq + t) * 69632: K and V as four balanced radix-256
 * int8 digit planes each plus per-key and per-channel metadata (exactattention_amd/csrc/
 * ea_params.h), the same tiles the prefill path otherwise slices into its workspace every step.
 * ea_hip_kv_digits_bytes: the cache size.
 * ea_hip_kv_digits_update: after keys key_begin[b] .. key_end[b] - 1 of each sequence b were
 *   written to the bf16 cache (and seq_len covers them), re-slice every tile that holds one of
 *   them, whole (keys at or past seq_len[b] slice as zero, so a tile is sliced again as it fills).
 *   key_begin, key_end: device int32[num_seqs]; max_new_keys >= every key_end[b] - key_begin[b]
 *   (sizes the grid); tiles at or past tiles_per_seq are skipped. Returns 0, -1 on bad arguments,
 *   -100 - e on a HIP error. Enqueue only (no sync).
 * Reference counterpart: the device slicing of the K/V caches, tc_slices_device /
 * tc_v_slices_device (src/exactattn/triton_kernels.py:1255-1280), which the reference reruns on
 * the whole cache at every launch. */
size_t ea_hip_kv_digits_bytes(int32_t num_seqs, int32_t num_kv_heads, int32_t tiles_per_seq);

/* KV append in one launch: rows i < n of k_new / v_new (row_elems uint16 each) written to rows
 * dst_rows[i] of the K and V pools (pool_rows rows of row_elems: a paged pool [pages, page_size,
 * Hkv, d] has rows of Hkv*d elements, row = page*page_size + slot), and block_table[bt_pos[j]] =
 * bt_val[j] for j < n_bt (entries at or past block_table_entries, and rows outside the pool, are
 * skipped). All pointers are device memory; dst_rows, bt_pos int64, bt_val int32. Enqueue only;
 * returns 0, -1 on bad arguments, -100 - e on a HIP error. A serving loop's append before its
 * attention call (with ea_hip_kv_digits_update when the digit cache is kept). Reference
 * counterpart: none; the reference's demo leaves its cache to transformers' DynamicCache
 * (scripts/spec_decode_demo.py:116-125). */
int ea_hip_kv_append(uint16_t* k_pool, uint16_t* v_pool, int64_t pool_rows, int64_t row_elems, const uint16_t* k_new,
                     const uint16_t* v_new, const int64_t* dst_rows, int64_t n, int32_t* block_table,
                     int64_t block_table_entries, const int64_t* bt_pos, const int32_t* bt_val, int64_t n_bt,
                     ea_stream_t stream);
int ea_hip_kv_digits_update(const ea_geometry* g, const ea_buffers* b, const int32_t* key_begin,
                            const int32_t* key_end, int32_t max_new_keys, void* kv_digits, int32_t tiles_per_seq,
                            ea_stream_t stream);

/* Library version string. */
const char* ea_hip_version(void);

#ifdef __cplusplus
}
#endif
#endif
