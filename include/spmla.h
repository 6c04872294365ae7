/* libspmla_gfx950.so: MI355X (gfx950) kernels for the dotsnote FP8 sparse-MLA attention path.
 *
 * Calling convention (the reference's, dotsnote/engine/arcstats_pkg/arcstats/offload_cuda2.py:21-90 and
 * csrc/offload_attn2.cu:2021-2104): raw device pointers into caller-owned buffers, element strides, a hipStream_t
 * passed as void*, an int return code (0 ok, a hipError_t value, or SPMLA_EARG -2 / SPMLA_EALIGN -3 /
 * SPMLA_ELIMIT -5 for rejected arguments). The library allocates nothing, never synchronizes the host and launches
 * only kernels on the caller's stream, so every entry point can be captured in a HIP graph. Strides are in elements
 * of the pointed-to type unless stated otherwise. bf16 tensors are passed as void* (uint16 bit patterns).
 *
 * Row formats: Row656 = [512 B e4m3fn latent | 4 x fp32 scale, one per 128 latent values | 64 x bf16 rope];
 *              Row576 = [512 B e4m3fn latent | 64 B e4m3fn rope], one per-tensor kv_scale;
 *              Row400 = the reference's compact e2m2b32 host row [256 B magnitude nibbles | 64 B sign bits |
 *                       16 x int8 block exponent (one per 32 latent values) | 64 B e4m3fn rope], one per-tensor
 *                       kv_scale; its latent values decode exactly to e4m3fn codes
 *                       (dotsnote/engine/arcstats_pkg/arcstats/offload_rowfmt.py:1-22).
 */
#ifndef SPMLA_H
#define SPMLA_H

#ifdef __cplusplus
extern "C" {
#endif

#define SPMLA_EARG (-2)
#define SPMLA_EALIGN (-3)
#define SPMLA_ELIMIT (-5)

/* KV-cache write: quantize and pack n tokens into rows at slots[i] (slot < 0 or >= R: skipped).
 * Row of a slot: cache + (slot / block_size) * block_stride + (slot % block_size) * row_bytes (block_stride in bytes).
 * fmt 0 = Row656 (per-128 absmax scales, kv_scale unused), fmt 1 = Row576 (clamp(x / kv_scale, +-448) -> e4m3),
 * fmt 2 = Row400 (clamp(x / kv_scale, +-448) -> sign + e2m2 with a power-of-two scale per 32 values; rope as Row576;
 * offload_rowfmt.py:81-129 _quant / _store_kernel, torch statement ref_quant / ref_pack :336-388).
 * kv_c: [n][512] bf16 (row stride kv_st), k_pe: [n][64] bf16 (row stride pe_st).
 * Replaces LayerOffload.store (dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:1131-1155, kernels :252-290)
 * and PortableSparseImpl.do_kv_cache_update (dsa_sm89.py:281-290); Row656 closed form
 * dotsnote/training/finetune/student.py:80-87, layout dotsnote/engine/vllm_patch/vllm/v1/hisparse/runtime.py:35-36. */
int spmla_cache_write(const void* kv_c, long long kv_st, const void* k_pe, long long pe_st, const long long* slots,
                      int n, void* cache, long long R, int block_size, long long block_stride, int fmt,
                      float kv_scale, void* stream);

/* Indexer key write: k [n][128] bf16 -> 132-byte rows [128 e4m3 codes | fp32 scale], scale = max(amax, 1e-4) / 448
 * (ue8m0 != 0: rounded up to a power of two). Rank-sharded store: slot s is owned by rank s % P as local row s / P
 * at store + (r / rows_per_block) * block_stride + (r % rows_per_block) * 132 (block_stride in bytes); P = 1 on one GPU.
 * Replaces ShardStore.write / _shard_write_kernel (dotsnote/engine/arcstats_pkg/arcstats/shard_indexer.py:42-60, :112-116). */
int spmla_index_key_write(const void* k, long long k_st, const long long* slots, int n, void* store,
                          long long R_local, int P, int rank, int rows_per_block, long long block_stride, int ue8m0,
                          void* stream);

/* Indexer logits: out[row][j] = min(sum_h w[row][h] * relu(q[row][h] . kcode) * kscale, 60000) for the key at
 * position pos = j * P + rank < ctx[row] (located through block_table[req[row]][pos / block_size]), -inf for
 * pos >= ctx (columns j < Lc; noinf != 0 leaves tiles wholly beyond ctx unwritten). q [rows][H][D] bf16 with H = 64,
 * D = 128; w [rows][H] fp32; out [rows][Lc] fp32 (out_dtype 0) or fp16 (out_dtype 1: each fp32 logit rounded to
 * nearest even, the reference's ARC_SHARD_F16OUT buffer, shard_indexer.py:28-29, :124; the 60000 clamp keeps it
 * finite); out_st in elements. ctx[row] <= block_size * (columns of the block table); R_local * P <= 2^31 - 1
 * (SPMLA_ELIMIT otherwise).
 * Replaces ShardStore.logits / _shard_logits_kernel and shard_logits_v2 'grp' / 'row8'
 * (dotsnote/engine/arcstats_pkg/arcstats/shard_indexer.py:63-91, :118-143; shard_logits_v2.py:15-138). */
int spmla_index_logits(const void* q, long long q_st, long long q_sh, const float* w, long long w_st,
                       const void* store, long long R_local, int rows_per_block, long long block_stride,
                       const int* block_table, long long bt_st, int block_size, const int* req, const int* ctx,
                       int rows, int H, int D, int Lc, int P, int rank, int noinf, void* out, long long out_st,
                       int out_dtype, void* stream);

/* Exact top-K per row over columns j < min(ctx[row], Lc) of logits [rows][Lc] (dtype 0: fp32, 1: fp16; lg_st in
 * elements): torch's order-preserving key (-0 < +0, NaN largest), equal values -> lower column; out[row][0..K) =
 * columns sorted by (value desc, column asc), -1 where the value is +-inf and for slots beyond the valid columns.
 * K <= 2048. The dtype argument is topk_local_launch's (csrc/topk_select.cu:250-262).
 * Replaces fast_topk.local + fast_topk.merge at P = 1 (dotsnote/engine/arcstats_pkg/arcstats/fast_topk.py:52-78;
 * csrc/topk_select.cu:251-286) and the torch.topk path of sharded_topk (shard_indexer.py:194-221). */
int spmla_topk(const void* logits, long long lg_st, const int* ctx, int rows, int Lc, int K, int* out,
               long long out_st, int dtype, void* stream);

/* Bytes of workspace spmla_topk_ws uses for rows x Lc (0 for invalid sizes): the per-row state, lists and histograms,
 * then the overflow lists (8 bytes per column) through which a narrowing level hands its boundary bin's keys to the
 * next level instead of that level reading the row again. */
long long spmla_topk_ws_bytes(int rows, int Lc, int K);

/* spmla_topk with the same result, spread over several workgroups per row: a histogram pass and a collect pass over
 * chunks of 8192 or more columns (at most 4 chunks per row), then one workgroup per row that resolves the boundary bin
 * and sorts. ws: device memory of spmla_topk_ws_bytes(rows, Lc, K) bytes (a smaller one without the overflow lists is
 * accepted: the second level then reads the row again), 16-byte aligned, any contents (every pass writes what the
 * next reads); calls that share a workspace must not overlap. Same replacement as
 * spmla_topk (fast_topk.local + merge at P = 1, dotsnote/engine/arcstats_pkg/arcstats/fast_topk.py:52-78;
 * csrc/topk_select.cu:251-286; shard_indexer.py:194-221). */
int spmla_topk_ws(const void* logits, long long lg_st, const int* ctx, int rows, int Lc, int K, int* out,
                  long long out_st, void* ws, long long ws_bytes, int dtype, void* stream);

/* spmla_index_logits (P = 1, rank 0) that also writes the first radix level of spmla_topk_ws into the top-k's
 * workspace ws (spmla_topk_ws_bytes(rows, Lc, K) bytes, 16-byte aligned): the logits workgroups cover the top-k's
 * column chunks and count the keys of the values they store in columns j < min(ctx[row], Lc), so the pass that would
 * re-read the logits for that histogram is not needed (spmla_topk_ws_prehist). Columns j < min(ctx, Lc) whose key
 * has no block-table entry are written -inf even with noinf != 0 (they are top-k columns). SPMLA_ELIMIT when a
 * chunk reaches 65536 columns (16-bit counts; Lc above 4 x 64512): use spmla_index_logits and spmla_topk_ws. The
 * reference computes the logits and then selects in separate calls (shard_indexer.py:63-91 then fast_topk.py:52-78 /
 * csrc/topk_select.cu:75-201 at P = 1, shard_indexer.py:194-221); the pair of entry points below is the same
 * computation with the selection's first pass done in the logits epilogue. */
int spmla_index_logits_hist(const void* q, long long q_st, long long q_sh, const float* w, long long w_st,
                            const void* store, long long R_local, int rows_per_block, long long block_stride,
                            const int* block_table, long long bt_st, int block_size, const int* req, const int* ctx,
                            int rows, int H, int D, int Lc, int noinf, void* out, long long out_st, int out_dtype,
                            void* topk_ws, long long ws_bytes, int K, void* stream);

/* spmla_topk_ws whose workspace already holds the first-level histograms of these logits (written by
 * spmla_index_logits_hist with the same rows, Lc, K, ctx and dtype, and no other use of the workspace in between):
 * the histogram pass is skipped; same result as spmla_topk_ws. */
int spmla_topk_ws_prehist(const void* logits, long long lg_st, const int* ctx, int rows, int Lc, int K, int* out,
                          long long out_st, void* ws, long long ws_bytes, int dtype, void* stream);

/* spmla_topk_ws without a caller workspace and without any allocation: the passes use the library's own
 * fixed device scratch (a file-scope array of spmla_topk_scratch_bytes() = 16 MiB per GPU, held from library load
 * until the process ends; its device address is looked up once per device on the first call there). Same result
 * as spmla_topk_ws (the overflow lists included when they fit the scratch). Sizes whose workspace without the
 * overflow lists exceeds the scratch return SPMLA_ELIMIT (e.g. 64 rows fit at any Lc up to 2^31). All calls on one GPU share the scratch: calls that overlap on one GPU (other streams,
 * other threads) race and must not be issued. The scratch keeps the last call's contents; the passes need no
 * particular initial contents. No counterpart in the reference: for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). */
long long spmla_topk_scratch_bytes(void);
int spmla_topk_scratch(const void* logits, long long lg_st, const int* ctx, int rows, int Lc, int K, int* out,
                       long long out_st, int dtype, void* stream);

/* fast_topk.local at rank `rank` of P: the row's valid columns are j < ceil((ctx[row] - rank) / P) (clipped to Lc);
 * the top kl of them by the same key and tie rule as spmla_topk go to pk[row] = [kl values fp32 | kl positions
 * j * P + rank as int32 bits] (pk row stride 2 * kl floats) in ascending column order; rows with fewer than kl valid
 * columns are padded with -inf values at positions s * P + rank. kl <= 2048. dtype 0: fp32 logits, 1: fp16 (the
 * payload values are the fp16 values widened to fp32).
 * Replaces topk_local_launch (dotsnote/engine/arcstats_pkg/arcstats/csrc/topk_select.cu:251-270, binding
 * fast_topk.py:52-66). */
int spmla_topk_local(const void* logits, long long lg_st, const int* ctx, int rows, int rank, int P, int Lc, int kl,
                     float* pk, int dtype, void* stream);

/* fast_topk.merge: allp [P][n][2 * kl] all-gathered local payloads (rank-major) -> out[row][0..kk) = positions of the
 * top kk of the P * kl candidates, ordered by (value desc, concatenation index asc), -1 where the value is +-inf;
 * out[row][kk..topk_tokens) = -1. kk <= min(P * kl, 2048).
 * Replaces topk_merge_launch (dotsnote/engine/arcstats_pkg/arcstats/csrc/topk_select.cu:272-286, binding
 * fast_topk.py:69-78). */
int spmla_topk_merge(const float* allp, int n, int P, int kl, int kk, int topk_tokens, int* out, long long out_st,
                     void* stream);

/* Request-local top-k positions -> global cache rows: rows[t][k] = block_table[req[t]][p / block_size] * stride_rows
 * + p % block_size for p = topk[t][k] >= 0 inside the table, else -1; counts[t] (optional) = valid entries.
 * Replaces vLLM's triton_convert_req_index_to_global_index (call sites dotsnote/engine/arcstats_pkg/arcstats/
 * dsa_sm89.py:314-315, :460-462, :467-469). T <= 65535. */
int spmla_rows_from_topk(const int* topk, long long tk_st, const int* req, const int* block_table, long long bt_st,
                         int bt_cols, int block_size, long long stride_rows, int T, int K, int* rows, long long r_st,
                         int* counts, void* stream);

/* Gather: dst row i (row stride dst_stride bytes) = src row rows[i] for 0 <= rows[i] < R, zero row otherwise.
 * src may be HBM or pinned host memory mapped into the device address space. row_bytes % 16 == 0.
 * Replaces LayerOffload.gather / _gather_rows_kernel (dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:
 * 293-306, :1157-1163). */
int spmla_gather(const void* src, long long R, int row_bytes, const long long* rows, int n, void* dst,
                 long long dst_stride, void* stream);

/* spmla_gather for a source in pinned host memory: the same result from a fixed grid of 64 workgroups that loops over
 * the rows. Reads over PCIe saturate the link from a quarter of the CUs, so kernels on other streams (the HBM-tier
 * attention of the same decode step) run beside it. Replaces the host-row path of LayerOffload.gather
 * (dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:1157-1163) and the miss fill's host reads
 * (offload_fill.py:204-248). */
int spmla_gather_pcie(const void* src, long long R, int row_bytes, const long long* rows, int n, void* dst,
                      long long dst_stride, void* stream);

/* Host-tier staging of a decode step: for each token t < T and k < counts[t] (clipped to K), dst row t * K + k
 * (row stride dst_stride bytes) = src row rows[t * r_st + k] (zero row when outside [0, R)); the other dst rows are
 * left as they are, except that dst row 0 is zeroed when counts[0] <= 0. rows / counts are spmla_tier_split's host
 * lists (compacted per token) and counts. Same 64-workgroup grid as spmla_gather_pcie. Replaces the miss copy of
 * the reference's tiered fill (dotsnote/engine/arcstats_pkg/arcstats/offload_fill.py:204-248; sparse_offload.py
 * :1157-1163 for one row). */
int spmla_gather_tiers(const void* src, long long R, int row_bytes, const int* rows, long long r_st, const int* counts,
                       int T, int K, void* dst, long long dst_stride, void* stream);

/* Row400 gather: dst row i (stride dst_stride bytes) = the GPU row of src Row400 row rows[i] (zero row when outside
 * [0, R)): dst_fmt 0 = Row656 (the decoded e4m3 codes, scales 1.0, rope widened to bf16: the same values, so the
 * attention reads it with the Row576 kv_scale), 1 = Row576 (the reference's GPU row, byte for byte). pcie != 0 runs
 * the fixed 64-workgroup grid of spmla_gather_pcie for a pinned host source. Replaces offload_rowfmt.gather /
 * _rows_kernel MODE 0 (dotsnote/engine/arcstats_pkg/arcstats/offload_rowfmt.py:163-185, :252-256, decode :131-160). */
int spmla_row400_gather(const void* src, long long R, const long long* rows, int n, void* dst, long long dst_stride,
                        int dst_fmt, int pcie, void* stream);

/* Gather of Row576 rows (the reference's per-tensor fp8 rows: 512 + 64 e4m3 codes, one kv_scale per tensor) into
 * Row656 staging rows for the attention: dst row i = src row rows[i] with its codes as they are, scales 1.0 and the
 * rope widened to bf16 (exact); a row id outside [0, R) gives a zero row. Attending the staging with the tensor's
 * kv_scale equals attending the Row576 rows. Replaces the Row576 row read of the portable attention
 * (PortableSparseImpl._run, dotsnote/engine/arcstats_pkg/arcstats/dsa_sm89.py:379-391, through
 * triton_bf16_mla_sparse_interface, vllm_patch/vllm/v1/attention/ops/xpu_mla_sparse.py:182-278). */
int spmla_row576_gather(const void* src, long long R, const long long* rows, int n, void* dst, long long dst_stride,
                        void* stream);

/* Row400 copy with decode: dst row dst_rows[i] (rows of dst_fmt's size) = the GPU row of src row src_rows[i]; pairs
 * with a side outside its range ([0, R_src), [0, R_dst)) are skipped. Fills GPU-format cache lines from compact host
 * rows. Replaces offload_rowfmt.refill / write_through (_rows_kernel MODE 1 and _wt_kernel, offload_rowfmt.py:187-249,
 * :258-267). */
int spmla_row400_copy(const void* src, long long R_src, const long long* src_rows, void* dst, long long R_dst,
                      const long long* dst_rows, int n, int dst_fmt, void* stream);

/* spmla_gather_tiers for Row400 host rows: the host-tier staging of a decode step with each row decoded to dst_fmt
 * (0 = Row656, 1 = Row576) on the way. Replaces the compact-row miss copy (offload_rowfmt.copy / _copy_kernel,
 * offload_rowfmt.py:187-221, :252-253). */
int spmla_row400_gather_tiers(const void* src, long long R, const int* rows, long long r_st, const int* counts, int T,
                              int K, void* dst, long long dst_stride, int dst_fmt, void* stream);

/* Compact Row400 lines in HBM decoded for the attention (the reference's compact GPU row cache, ARC_OFFLOAD_CCACHE,
 * whose loaders decode the lines in shared memory, csrc/offload_attn2.cu:210-256): dst row t * K + k = the dst_fmt row
 * (0 = Row656, 1 = Row576) of src row rows[t * r_st + k] (zero row when outside [0, R)) for k < counts[t] (counts
 * NULL: every k < K); other dst rows untouched. src in HBM: 16 lanes per row, each decoding one 32-value block. */
int spmla_row400_decode_tiers(const void* src, long long R, const int* rows, long long r_st, const int* counts, int T,
                              int K, void* dst, long long dst_stride, int dst_fmt, void* stream);

/* Dynamic W-way HBM row cache, bookkeeping of one decode step (no row copies). Host row h lives in set h % S
 * (S = C / W), in any line st * W + w with tag[line] == h (-1 empty). For the selected rows idx [T][K] (invalid =
 * outside [0, R)): entries whose row is cached pin their line for the step; each distinct missing row takes a ticket
 * in its set and the ticket-th unpinned way counted round-robin from rr[set] (its tag is set to the row), or, with no
 * unpinned way left, spill row C + k (k < cap) or the host (-2); rr[set] advances by min(tickets, W). res [T][K]
 * (stride res_st) = the pool row holding each entry's row (line or C + k), -2 host, -1 invalid. The miss list
 * (miss_rows, miss_dst: >= T * K entries) and state (int[4]: epoch, misses, spill rows used, hits) feed
 * spmla_wcache_fill. Caller-owned state, zero-initialized once: tag -1, rr / cnt / pin / state / claim 0; claim and
 * rdst hold one int per host row (the epoch of the row's last miss, the pool row it got), so no buffer is cleared
 * between steps. Which ways the misses of a set take, and which misses of an overfull set spill, follow the order of
 * the device atomics. two = 1: two-choice placement (the reference's ARC_OFFLOAD_TWO_CHOICE, offload_fill.py:16-23,
 * :136-165, :255-303): row h may also live in set ((h * 2654435761) >> 12) % S; entries that miss the first set look
 * there (a hit pins it), and a miss with no unpinned way for its ticket in the first set takes a ticket in the second
 * before it spills. The same `two` must be passed to every call on one cache (spmla_wcache_invalidate included).
 * Replaces the reference's W-way cache step (_sa_prefill and _sa_scan / _sa_fill / _sa_advance / _sa_resolve
 * kernels, dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:677-770, :1595-1622; epoch-tagged miss table
 * offload_fill.py:1-45). */
int spmla_wcache_step(const int* idx, long long idx_st, int T, int K, long long R, int* tag, int C, int W, int* rr,
                      int* cnt, int* pin, int* claim, int* rdst, long long* miss_rows, long long* miss_dst, int* state,
                      int cap, int two, int* res, long long res_st, void* stream);

/* spmla_wcache_step in two launches groups, so that the row copies can start before the resolution: _place runs the
 * step's lookup and placement (the miss list and the tags are final after it; spmla_wcache_fill may follow on
 * another stream), _resolve writes res and advances the round-robin pointers. Same arguments and results. */
int spmla_wcache_place(const int* idx, long long idx_st, int T, int K, long long R, int* tag, int C, int W, int* rr,
                       int* cnt, int* pin, int* claim, int* rdst, long long* miss_rows, long long* miss_dst, int* state,
                       int cap, int two, void* stream);
int spmla_wcache_resolve(const int* idx, long long idx_st, int T, int K, long long R, int* tag, int C, int W, int* rr,
                         int* cnt, int* pin, int* claim, int* rdst, long long* miss_rows, long long* miss_dst,
                         int* state, int cap, int two, int* res, long long res_st, void* stream);

/* The step's row copies: for each miss m < state[1] with miss_dst[m] >= 0, pool row miss_dst[m] = host row
 * miss_rows[m]. host_fmt / pool_fmt: 0 / 0 Row656 bytes into Row656 lines; 2 / 0 a compact Row400 row decoded into a
 * Row656 line; 2 / 2 the Row400 bytes as they are into compact Row400 lines (the reference's compact GPU row cache,
 * ARC_OFFLOAD_CCACHE). n_max bounds the miss count (T * K of the step). 64 workgroups, rows streamed two per wave
 * (the PCIe gather). Replaces the copy half of the reference's fill (_sa_fill_kernel sparse_offload.py:722-760; the
 * split fill's gather, offload_fill.py:311-333). */
int spmla_wcache_fill(const void* host, long long R, int host_fmt, int pool_fmt, const long long* miss_rows,
                      const long long* miss_dst, const int* state, int n_max, void* pool, long long R_pool,
                      void* stream);

/* Clear the lines that cache rows slots[i] (a rewritten host row must not be served stale); two = 1 also clears
 * the rows' second sets. Replaces _sa_invalidate_kernel (sparse_offload.py:782-789) and, for two-choice placement,
 * _invalidate2_kernel (offload_fill.py:296-308). */
int spmla_wcache_invalidate(const long long* slots, int n, long long R, int* tag, int C, int W, int two, void* stream);

/* Tier split by resolution: per token, entries with res >= 0 -> hbm_idx (the pool row), res == -2 -> host_idx (the
 * entry's host row idx[t][k]); both compacted in order, padded with -1 to K, counts per token. The host tier of a
 * cache whose spill area overflowed (the reference's attention reads res == -1 entries from the host,
 * csrc/offload_attn2.cu:1610-1995). */
int spmla_split_res(const int* idx, long long idx_st, const int* res, long long res_st, int T, int K, int* hbm_idx,
                    long long hbm_st, int* hbm_cnt, int* host_idx, long long host_st, int* host_cnt, void* stream);

/* Split of a cache step's resolutions by hit: per token, entries whose line was a hit of the step (pin[line] equals
 * the step's epoch, state[0]) -> hit_idx, the other entries with res >= 0 (rows the step's fill brings in) ->
 * fresh_idx; both as pool rows, compacted in order, padded with -1, with counts per token. The attention over the
 * hits can then run while spmla_wcache_fill copies the misses in, and the attention over the fresh rows merges it
 * (spmla_attn_merge). Replaces the reference's overlapped fill, where the attention waits on per-row pending marks
 * (offload_fill.py:33-38, ARC_OFFLOAD_OVERLAP). */
int spmla_wcache_split(const int* res, long long res_st, int T, int K, const int* pin, int C, const int* state,
                       int* hit_idx, long long hit_st, int* hit_cnt, int* fresh_idx, long long fresh_st, int* fresh_cnt,
                       void* stream);

/* Row copy: dst row dst_rows[i] = src row src_rows[i] (pairs with an out-of-range side skipped); fills the HBM hot-row
 * cache from the host pool. Replaces the row-cache fill copies (offload_fill.py:311-333, csrc/offload_attn.cu:522-584). */
int spmla_copy_rows(const void* src, long long R_src, const long long* src_rows, void* dst, long long R_dst,
                    const long long* dst_rows, int row_bytes, int n, void* stream);

/* Tier split of the selected rows: for each token t, valid host rows h = idx[t][k] (0 <= h < R) with rowmap[h] >= 0
 * go to hbm_idx[t] as cache line rowmap[h], the others to host_idx[t] as h; both compacted in order, padded with -1
 * to K; hbm_cnt[t] / host_cnt[t] = lengths. Replaces the hit / miss resolution of the row cache
 * (dotsnote/engine/arcstats_pkg/arcstats/offload_fill.py:204-248, sparse_offload.py:454-456, :756-778). */
int spmla_tier_split(const int* idx, long long idx_st, int T, int K, const int* rowmap, long long R, int* hbm_idx,
                     long long hbm_st, int* hbm_cnt, int* host_idx, long long host_st, int* host_cnt, void* stream);

/* Prefill compact stage: sidx [M][K] positions into rows[0..tot) (-1 = none) -> sel[0..U) = rows of the distinct
 * selected positions in ascending order, sidx2 = positions into sel (-1 kept), *U on the device.
 * workspace: 2 * ceil(tot / 32) uint32, caller-owned. Replaces compact_stage (dsa_sm89.py:27-35). */
int spmla_compact_stage(const long long* rows, int tot, const int* sidx, long long s_st, int M, int K, void* workspace,
                        long long* sel, int* U, int* sidx2, long long s2_st, void* stream);

/* Sparse-MLA attention over Row656 rows. q [T][H][576] bf16 (16-byte aligned rows), pool [R] Row656 rows,
 * idx [T][K] int32 rows of the pool (invalid = outside [0, R)), kcount (optional) [T]: only the first kcount[t]
 * entries are read. s = sm_scale * kv_scale * q . row; o = kv_scale * softmax(s) V_latent; lse = ln sum exp(s)
 * (-inf and o = 0 for a token with no valid entry).
 * opart == NULL (S == 1): out [T][H][512] bf16 (strides o_st, o_sh), lse [T][H] fp32 (stride lse_st).
 * opart != NULL (required for S > 1): the K entries are cut into S splits; opart [S][T][H][512] fp32 (normalized)
 * and lsepart [S][T][H] receive per-split partials for spmla_lse_merge (S = 1: one fp32 partial, e.g. per tier);
 * out / lse are not written then. Any K. Two kernels serve it with the same results up to fp32 summation order:
 * launches of at most 512 (token, split, 32-head group) work items run 32 heads per workgroup (decode batches),
 * longer ones 128 heads per workgroup (prefill chunks; there ceil(ceil(K / S) / 32) * 32 > 2048 falls back to the
 * first kernel).
 * Replaces LayerOffload.attend's decode kernels (oa2_v2_launch dotsnote/engine/arcstats_pkg/arcstats/csrc/
 * offload_attn2.cu:2021-2104, offload_split_launch csrc/offload_attn.cu:1155-1200, _sparse_mla_offload_split_kernel
 * sparse_offload.py:419-516) and triton_bf16_mla_sparse_interface (vllm_patch/.../ops/xpu_mla_sparse.py:182-278),
 * extended by the LSE output. */
int spmla_attn_splitk(const void* q, long long q_st, long long q_sh, const void* pool, long long R,
                      const int* idx, long long idx_st, int K, const int* kcount, int T, int H, float sm_scale,
                      float kv_scale, int S, void* out, long long o_st, long long o_sh, float* lse,
                      long long lse_st, float* opart, float* lsepart, void* stream);

/* spmla_attn_splitk over Row576 rows, the plugin's per-tensor "fp8" cache: pool [R] rows of 512 latent + 64 rope
 * e4m3 codes (no per-group scales), every code times the tensor's kv_scale. Same arguments, outputs and results
 * (o = kv_scale * softmax(s) codes_latent, s = sm_scale * kv_scale * q . codes); S > 1 needs opart / lsepart (the
 * fp32 partials for spmla_lse_merge). Any K; one kernel (32 heads per workgroup) serves every launch.
 * Replaces triton_bf16_mla_sparse_interface over the fp8 per-tensor rows (PortableSparseImpl._run,
 * dotsnote/engine/arcstats_pkg/arcstats/dsa_sm89.py:379-391, kernel vllm_patch/.../ops/xpu_mla_sparse.py:77-161). */
int spmla_attn576(const void* q, long long q_st, long long q_sh, const void* pool, long long R, const int* idx,
                  long long idx_st, int K, const int* kcount, int T, int H, float sm_scale, float kv_scale, int S,
                  void* out, long long o_st, long long o_sh, float* lse, long long lse_st, float* opart,
                  float* lsepart, void* stream);

/* Bytes of the workspace spmla_attn needs for T tokens, H heads and S splits (0 for S = 1; -1 for bad sizes). */
long long spmla_attn_ws_bytes(int T, int H, int S);

/* spmla_attn_splitk with the bf16 out + lse for any S in 1 .. 8: the S splits of a (token, group of 128 heads) merge
 * in the kernel -- each writes its normalized partial (f16, with a power-of-two exponent per head that keeps it in
 * range) and lse to ws, and the last split to finish merges all of them (weights e^(lse_s - M) / Z) into out / lse.
 * ws: spmla_attn_ws_bytes(T, H, S) bytes, 256-byte aligned. Its first C = 4 * T * ceil(H / 128) bytes (rounded up
 * to a multiple of 256) are the launch's counters and must be zero when it starts; the kernel leaves them zero, and
 * the bytes past them are scratch. So a workspace zero-filled once serves launches that run one after another,
 * except that a launch with a larger C than the previous launch on the same workspace needs the bytes from the
 * previous C to its own C zeroed first. Launches that may overlap need workspaces of their own. out 16-byte aligned
 * rows give 16-byte stores. S > 8 or ceil(ceil(K / S) / 32) * 32 > 2048: SPMLA_ELIMIT. S = 1 is spmla_attn_splitk
 * (ws unused).
 * Replaces the split-K decode launch with its partial combine (oa2_v2_launch dotsnote/engine/arcstats_pkg/arcstats/
 * csrc/offload_attn2.cu:2021-2104; _sparse_mla_offload_split_kernel + _combine_kernel sparse_offload.py:419-538). */
int spmla_attn(const void* q, long long q_st, long long q_sh, const void* pool, long long R, const int* idx,
               long long idx_st, int K, const int* kcount, int T, int H, float sm_scale, float kv_scale, int S,
               void* out, long long o_st, long long o_sh, float* lse, long long lse_st, void* ws, long long ws_bytes,
               void* stream);

/* spmla_attn_splitk (S = 1) whose result is merged with a prior partial of the same tokens and heads before the bf16
 * write: prior_o [T][H][512] fp32 normalized (strides po_st, po_sh; 16-byte aligned), prior_lse [T][H] (stride
 * pl_st, natural log). out = w o + w' prior_o with w = e^lse / (e^lse + e^lse'), w' = e^lse' / (e^lse + e^lse'),
 * lse_out = ln(e^lse + e^lse'); both -inf -> o = 0, lse = -inf. The host-tier attention of a decode step merges the
 * HBM tier's partial this way, in place of spmla_lse_merge over two partials (the reference's tier combine,
 * dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:519-538, fused into the second tier's kernel). */
int spmla_attn_merge(const void* q, long long q_st, long long q_sh, const void* pool, long long R, const int* idx,
                     long long idx_st, int K, const int* kcount, int T, int H, float sm_scale, float kv_scale,
                     const float* prior_o, long long po_st, long long po_sh, const float* prior_lse, long long pl_st,
                     void* out, long long o_st, long long o_sh, float* lse, long long lse_st, void* stream);

/* LSE merge of n partial results (splits or tiers): part i of (t, h) at parts + i*o_ps + t*o_st + h*o_sh (512 values,
 * fp32 or bf16), lse[i*l_ps + t*l_st + h]. o = sum_i exp(lse_i - L) o_i, L = ln sum_i exp(lse_i); all parts -inf ->
 * o = 0, L = -inf. out bf16 and/or out_f32 (same strides), lse_out optional.
 * Replaces _combine_kernel (dotsnote/engine/arcstats_pkg/arcstats/sparse_offload.py:519-538) and the
 * merge_attn_states call (vllm_patch/vllm/model_executor/layers/attention/sparse_mla_attention.py:1091-1097). */
int spmla_lse_merge(const void* parts, int parts_bf16, long long o_ps, long long o_st, long long o_sh,
                    const float* lse, long long l_ps, long long l_st, int n, int T, int H, void* out,
                    long long out_st, long long out_sh, float* out_f32, float* lse_out, long long lo_st,
                    void* stream);

/* Per-head matmul on FP8 block-scaled weights: C[n][b][j] = sum_k A[n][b][k] * bf16(fp32(e4m3(W[n][j][k]) * S)),
 * S = s[n][j][k / 128] (scale_k = 1) or s[n][k][j / 128] (scale_k = 0), fp32 accumulation. A bf16 (strides sa_*),
 * W e4m3 codes (strides sw_*), s fp32 (strides ss_n, ss_0, ss_1 over its three dimensions), C bf16 or fp32 (out_f32)
 * with strides sc_*. K % 8 == 0. Contiguous, 16-byte aligned operands with K % 16 == 0 take the LDS-staged kernel.
 * Replaces _bmm_fp8_kernel / bmm_fp8 (dotsnote/engine/arcstats_pkg/arcstats/mla_fp8.py:22-67), which serves MLA's
 * absorbed W_UK_T and W_UV products (its _TorchProxy.bmm, :121-132). */
int spmla_bmm_fp8(const void* a, long long sa_n, long long sa_b, long long sa_k, const void* w, long long sw_n,
                  long long sw_j, long long sw_k, const float* s, long long ss_n, long long ss_0, long long ss_1,
                  int scale_k, void* c, long long sc_n, long long sc_b, long long sc_j, int out_f32, int N, int B,
                  int J, int K, void* stream);

/* The decode query of the sparse attention in one launch: q[t][h][0:512] = q_nope[t][h][0:128] @ W_UK_T[h] on the
 * FP8 form (codes [H][512][128] contiguous, scales [H][128][4] fp32, scale over k), q[t][h][512:576] = q_pe[t][h]
 * copied bit for bit. q rows 16-byte aligned (strides q_st, q_sh, in elements, multiples of 8).
 * Replaces the qcat patch's bmm into the first columns of the concatenated query plus the q_pe copy
 * (dotsnote/engine/arcstats_pkg/arcstats/qcat.py:20-28), with mla_fp8's FP8 weights (mla_fp8.py:77-109). */
int spmla_mla_query(const void* q_nope, long long qn_st, long long qn_sh, const void* q_pe, long long qp_st,
                    long long qp_sh, const void* w_uk, const float* s_uk, int T, int H, void* q, long long q_st,
                    long long q_sh, void* stream);

/* Indexer key write into vLLM's paged indexer key cache in its SHUFFLE layout: key at slot = block * block_size + t
 * (block_size % 16 == 0, block b at cache + b * block_stride bytes): its 128 e4m3 codes in 16-token x 16-byte tiles,
 * code d at (t / 16) * 2048 + (t % 16) * 16 + (d / 16) * 256 + d % 16, its fp32 scale at block_size * 128 + 4 t; the
 * quantization of spmla_index_key_write (s = max(amax, 1e-4) / 448, UE8M0 option). Slots < 0 or beyond the cache are
 * skipped. The layout is the one the reference's paged reader addresses (dotsnote/engine/arcstats_pkg/arcstats/
 * dsa_sm89.py:63-66); the writer it pairs with is vLLM's indexer cache insert (compiled, not in the tree). */
int spmla_index_key_write_shuffle(const void* k, long long k_st, const long long* slots, int n, void* cache,
                                  long long num_blocks, int block_size, long long block_stride, int ue8m0,
                                  void* stream);

/* spmla_index_logits over the SHUFFLE cache (P = 1, no 60000 clamp): out[row][j] = sum_h w[row][h] *
 * relu(q[row][h] . kcode) * kscale for positions j < ctx[row] (key block block_table[req[row]][j / block_size]),
 * -inf beyond (noinf: left unwritten). H = 64, D = 128, q bf16.
 * Replaces paged_mqa_logits_triton / _paged_logits_kernel (dotsnote/engine/arcstats_pkg/arcstats/dsa_sm89.py:41-94),
 * the decode logits of the reference's default indexer path; the host wrapper builds req / ctx for next_n > 1. */
int spmla_paged_mqa_logits(const void* q, long long q_st, long long q_sh, const float* w, long long w_st,
                           const void* cache, long long num_blocks, int block_size, long long block_stride,
                           const int* block_table, long long bt_st, const int* req, const int* ctx, int rows, int H,
                           int D, int Lc, int noinf, float* out, long long out_st, void* stream);

/* Prefill indexer logits over gathered keys: out[m][n] = sum_h w[m][h] * relu(q[m][h] . kcode[n]) * kscale[n] for
 * ks[m] <= n < ke[m], -inf for the other n < N (no clamp). Key n's 128 e4m3 codes at k + n * k_st bytes, its fp32
 * scale kscale[n]. H = 64, D = 128, q bf16.
 * Replaces mqa_logits_triton / _mqa_logits_kernel (dotsnote/engine/arcstats_pkg/arcstats/dsa_sm89.py:96-133). */
int spmla_mqa_logits(const void* q, long long q_st, long long q_sh, const float* w, long long w_st, const void* k,
                     long long k_st, const float* kscale, int N, const int* ks, const int* ke, int M, int H, int D,
                     float* out, long long out_st, void* stream);

/* Request-packed MTP decode, the row list: for request r (tokens cu[r] .. cu[r + 1], or r * ql .. + ql clipped to
 * T), u[r][0 .. cnt[r]) = the distinct rows 0 <= row < R of those tokens' top-k lists
 * (idx [T][topk], row stride idx_st), mk[r][i] = bit j set when token j selected row u[r][i]; ordered by mask
 * descending, then by the position j * topk + k of the row's first occurrence; u[r][cnt .. nmax) = -1.
 * nmax >= (tokens used) * topk, R < 2^26 - 1, topk <= 2048. A request holds at most 6 tokens: ql > 6 is
 * SPMLA_EARG; with cu the caller guarantees it (the boundaries stay on the device; the Python wrapper checks them).
 * Replaces pk_union_kernel (dotsnote/engine/arcstats_pkg/arcstats/csrc/offload_attn.cu:586-698, ARC_OFFLOAD_CUDA_PK). */
int spmla_mtp_union(const int* idx, long long idx_st, int T, int ql, const int* cu, int nreq, long long R, int topk,
                    int nmax, int* u, unsigned char* mk, int* cnt, void* stream);

/* Request-packed MTP decode attention over the union rows of spmla_mtp_union (u, mk, cnt; row capacity nmax): a
 * workgroup's 32 query columns are tpg (1, 2, 4, 8) tokens of one request x 32 / tpg heads, so each union row is
 * loaded and converted once for all of them; a column's softmax uses only the rows its token's mask holds. Request
 * r = tokens cu[r] .. cu[r + 1] (or r * ql .. + ql clipped to T), at most 6 of them (ql > 6: SPMLA_EARG). Results
 * and outputs as spmla_attn_splitk for each token (S splits of the union with fp32 partials, or S = 1 with the
 * bf16 out + lse), up to the fp32 summation order of the rows.
 * Replaces pk_attn_kernel (dotsnote/engine/arcstats_pkg/arcstats/csrc/offload_attn.cu:700-1153). */
int spmla_attn_packed(const void* q, long long q_st, long long q_sh, const void* pool, long long R, const int* u,
                      const unsigned char* mk, const int* cnt, int nmax, const int* cu, int ql, int nreq, int T,
                      int H, int tpg, float sm_scale, float kv_scale, int S, void* out, long long o_st,
                      long long o_sh, float* lse, long long lse_st, float* opart, float* lsepart, void* stream);

/* Top-k overlap of L layers' selections for n query rows: for layers a != b, hits[(a L + b) n + i] = number of valid
 * entries (>= 0) of layer b's row i that also occur in layer a's row i (symmetric for duplicate-free rows; the
 * diagonal is not written); nvalid[a n + i] = valid entries of layer a's row i. Entry k of layer l, row i at
 * sets[l s_l + i s_r + k]. K <= 2048.
 * Replaces TopkOverlap._accumulate's sort / searchsorted intersection (dotsnote/engine/arcstats_pkg/arcstats/
 * index_share.py:109-130), the statistic behind cross-layer top-k sharing (ARC_INDEX_SHARE). */
int spmla_topk_overlap(const int* sets, long long s_l, long long s_r, int L, int n, int K, int* hits, int* nvalid,
                       void* stream);

/* Build identification string (static storage). */
const char* spmla_version(void);

/* Host-side self-test hook: the e4m3fn encoder the kernels use, run on the CPU (no GPU call). */
void spmla_host_e4m3_encode(const float* x, unsigned char* out, long long n);

#ifdef __cplusplus
}
#endif

#endif /* SPMLA_H */
