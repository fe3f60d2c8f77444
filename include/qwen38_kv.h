/*
 * qwen38_kv.h -- C ABI of the MI355X (gfx950) quantized KV-cache path: the append/evict half (q8 window ring plus the
 * 4..8-bit packed long-term store, optional 256-point Walsh-Hadamard rotation) and the gather+attention half (split-K
 * GQA decode attention over the mixed store, 1..8 query tokens, paged multi-sequence).
 *
 * Conventions (the reference's C API, capi.cpp:190-263): an opaque handle; int status, >= 0 success, -1 error with the
 * message in the thread-local mk_last_error(); no exception crosses the ABI; caller-owned output buffers with a cap,
 * and cap 0 / NULL returns the count needed.  Device pointers are HIP device addresses already resident in HBM;
 * `stream` is a hipStream_t (NULL: the default stream).  One handle is not thread-safe: calls on it are serialised by
 * the caller, as with the reference's engine.  The attend and prefill calls of one handle share its split-K workspace:
 * issue them on one stream (or order the streams between calls), or their partials overwrite each other.  The
 * workspace grows on demand (by at least 1.5 times); a buffer it outgrows is kept, not freed, until mk_free, so a HIP
 * graph captured over an earlier call stays valid after a larger call (its replays keep using the old, smaller
 * buffer; a graph replay and an eager call of one handle must still not overlap).  The kept buffers together stay
 * below twice the live workspace.
 *
 * Shapes: NKV = 4 kv heads, NH = 24 query heads (GQA 6), head dim 256, up to 17 attention slots (layers), up to 8
 * query tokens per attend call, up to 8 sequences per attend call.
 */
#ifndef QWEN38_KV_H
#define QWEN38_KV_H

#ifdef __cplusplus
extern "C" {
#endif

/* Last error of this thread.  Replaces mk_last_error, capi.cpp:263. */
const char * mk_last_error(void);

/*
 * Create a KV store.  Replaces the KV block of mk_new_mtp / MKEngine construction (capi.cpp:266, loader.cu:1329-1510).
 *   kv_spec   the MK_KV grammar: comma-separated <K|V|*><slot>=<4..8>[r] (slot 0..n_layers-1, * or empty: all;
 *             r: stored Walsh-Hadamard rotated); NULL or "" = every side q8 (loader.cu:1329-1365)
 *   win       MK_KV_WIN: low-bit sides keep their newest >= win positions as q8 in a ring of
 *             (ceil(win/640)+1)*640+32 rows per kv head (loader.cu:1469-1510); 0 = no window
 *   win_all   MK_KV_WIN_ALL: rings for the q8 sides too (test knob, loader.cu:1487-1490)
 *   n_layers  attention slots, 1..17
 *   n_seq     sequences (lanes), 1..64
 *   ctx       positions per sequence
 *   page      positions per page, a multiple of 32; 0 = one contiguous page per sequence (the reference's
 *             [kv head][ctx][row] layout)
 *   n_pages   pages in the shared pool; 0 = n_seq * ceil(ctx / page).  Each sequence starts with the identity table
 *             over its own range of pages (when the pool is large enough).
 * Returns NULL on error (mk_last_error).
 */
void * mk_kv_new(const char * kv_spec, int win, int win_all, int n_layers, int n_seq, int ctx, int page, int n_pages);

/* Free a store (replaces mk_free, capi.cpp:418).  NULL is a no-op. */
void mk_free(void * h);

/* Set the page table of one sequence: logical page i -> physical page pages[i] (host array, n <= ceil(ctx/page)).
 * No counterpart in the reference (its lanes are contiguous, lanes.cu:290-345); added for paged multi-sequence. */
int mk_kv_set_pages(void * h, int seq, const int * pages, int n);

/*
 * Append T positions pos .. pos+T-1 of sequence seq for slots layer0 .. layer0+n_layers-1.  k, v: device arrays
 * [T][n_layers][4][256] of fp32 (dtype 0) or fp16 (dtype 1), the rows after RMSNorm/RoPE.  Each row is stored in its
 * side's format (optionally rotated) and, for sides with a window, as q8 in the ring.  Replaces the kv_store step of
 * mk_step / mk_prefill (capi.cpp:508-554 -> qwen38_mk.cu:2099-2116, 2955-2985).  Asynchronous on `stream`.
 */
int mk_kv_append(void * h, int seq, int layer0, int n_layers, int pos, int T, const void * k, const void * v, int dtype, void * stream);

/*
 * Decode attention for n_seq sequences (seqs[i], context lens[i] after this call's T rows) over slots layer0 ..
 * layer0+n_layers-1.  q: device [n_layers][n_seq][T][24][256] fp32 (after RMSNorm/RoPE, before the 1/16 scale);
 * out: device, same shape, the attention output before the output gate (V un-rotated when V is stored rotated).
 * Token t of a sequence sees positions <= lens[i] - T + t.  The T rows must share one 640-position window bucket
 * (att_cap_T, mk_shared.cuh:288-291; see mk_kv_cap_T).  Replaces attn_core + attn_combine of mk_step
 * (qwen38_mk.cu:4568-4700).  Asynchronous on `stream`.
 */
int mk_kv_attend(void * h, int layer0, int n_layers, int n_seq, const int * seqs, const int * lens, int T, const float * q, float * out,
                 void * stream);

/*
 * Prefetch for a later mk_kv_attend with the same (layer0, n_layers, seqs, lens, T): the first `tiles` (1..64) tiles
 * of every wave slice of every segment are read by one workgroup per segment, placed on the XCD that the attention's
 * workgroups for that segment (both row batches at T = 5..8) run on, so the tiles sit in that XCD's L2 (and in the
 * last-level cache).  Issue it on another
 * stream beside independent work (the layer's projections) before the attention; it writes nothing.  Same checks as
 * mk_kv_attend.  Replaces the L2 prefetch of the first KV lines in attn_proj (pf_l2, qwen38_mk.cu:2600-2621).
 */
int mk_kv_prefetch(void * h, int layer0, int n_layers, int n_seq, const int * seqs, const int * lens, int T, int tiles, void * stream);

/*
 * mk_kv_append followed by mk_kv_attend in one launch: the T new rows of every sequence (positions lens[i] - T ..
 * lens[i] - 1; k, v device [n_seq][T][n_layers][4][256] of fp32 (dtype 0) or fp16 (dtype 1), rows after RMSNorm/RoPE)
 * are stored by the attention kernel itself -- by the wave whose tiles hold them, before those tiles are copied --
 * and the queries attend over the store including them.  Same stored bytes and outputs as the two calls; one launch
 * fewer per decode slot (the reference stores the step's K/V inside its attention work items, qwen38_mk.cu:2915-2923,
 * 3512-3519, 4126-4133).  lens[i] - T must not exceed the stored length (no gap).
 */
int mk_kv_append_attend(void * h, int layer0, int n_layers, int n_seq, const int * seqs, const int * lens, int T, const void * k, const void * v,
                        int dtype, const float * q, float * out, void * stream);

/*
 * mk_kv_attend that allocates nothing: no hipMalloc / hipFree, no host heap.  No counterpart in the reference; for
 * callers that cannot allocate (code under HIP graph capture, tight serving loops).  The segment partials go to a
 * 64 MiB device array the library holds on each GPU it runs on (looked up on the first call on a device, which must be
 * the store's device); a call whose partials need more fails with -1 and a message.  The partials take 1,032 bytes per
 * (query row, split-K segment), at most 128 segments per kv head: 16 layers of one sequence at T = 1, or 2 layers at
 * T = 8, fit at any context.  Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (several streams, threads or stores) race.  Nothing in it needs
 * clearing: each call writes every partial it reads.  Same arguments, outputs and bits as mk_kv_attend.
 */
int mk_kv_attend_noalloc(void * h, int layer0, int n_layers, int n_seq, const int * seqs, const int * lens, int T, const float * q,
                         float * out, void * stream);

/*
 * mk_kv_attend followed by the combine epilogue (qwen38_mk.cu:4686-4688): out = y / (1 + exp(-gate)) with gate a
 * device array shaped like q, and, when q32a / q32b / q32meta are given (all three or none), out in the o_proj
 * activation units of q32_store (qwen38_mk.cu:283-307): per token row of 24 x 256 outputs, 32-value blocks
 * j = 8 head + k quantised to int8 (amax / 127, round half away from zero); unit gi = 8 head + 2 (k / 2) + half holds
 * 16 bytes of an even block in q32a [..][192][16] and of an odd block in q32b, and q32meta [..][192][4] = fp16 scale
 * of the q32a / q32b block, int16 sum of the q32a / q32b half.  Shapes [n_layers][n_seq][T][...].
 */
int mk_kv_attend_gated(void * h, int layer0, int n_layers, int n_seq, const int * seqs, const int * lens, int T, const float * q,
                       const float * gate, float * out, void * q32a, void * q32b, unsigned short * q32meta, void * stream);

/*
 * The Q/K prep as a fused producer (qwen38_mk.cu:2843-2880, 2903-2910; prefill.cuh:986-1000): RMSNorm over each
 * 256-value head row (eps 1e-6, per-slot weight) and NeoX RoPE on values 0..63 (pair i, i+32) from the store's RoPE
 * table.  The table is [rows][32] float2 (cos, sin) in device memory: the caller's (e.g. the reference's rewritten
 * image rows, engine.cu:30-62) via mk_kv_set_rope(h, table, rows), or with table = NULL the text table the reference
 * builds (loader.cu:1252-1258: p * 1e7^(-2i/64) in double, rounded to float), ctx rows, built once by the store.
 * Exactness: the prep's arithmetic order is this library's own (FMA-chain partial sums, a 64-lane butterfly, 1/sqrtf);
 * the reference's uses rsqrtf and a 32-lane reduction.  Prepped values therefore differ from the reference's by a few
 * ulp, so K rows stored through mk_kv_append_prep / mk_kv_prefill_prep are bit-exact only against a restatement of
 * this order (oracle kvo_qk_prep), not against the reference's stored bytes; the rows of mk_kv_append (already prepped
 * input) are bit-exact against the reference's quantizers.
 */
int mk_kv_set_rope(void * h, const void * table, int rows);

/*
 * mk_kv_append of raw K rows: k [T][n_layers][4][256] fp32 before the k-norm / RoPE, v as for mk_kv_append (fp32),
 * k_norm device [n_layers][256] weights; the K row of position p is normed and rotated by table row p inside the
 * append kernel (the kv_store producer of mk_step, qwen38_mk.cu:2903-2911).
 */
int mk_kv_append_prep(void * h, int seq, int layer0, int n_layers, int pos, int T, const float * k, const float * v, const float * k_norm,
                      void * stream);

/*
 * mk_kv_attend_gated on the raw q_proj output: qg device [n_layers][n_seq][T][24][512], per head 256 query values
 * before the q-norm / RoPE followed by 256 gate values (the reference's qbuf, qwen38_mk.cu:2836, 4640);
 * q_norm device [n_layers][256].  Query row t of a sequence of length L is rotated by table row L - T + t.  out and
 * the optional q32 set as for mk_kv_attend_gated.  This is the attention of one mk_step slot from q_proj to o_proj.
 */
int mk_kv_attend_prep(void * h, int layer0, int n_layers, int n_seq, const int * seqs, const int * lens, int T, const float * qg,
                      const float * q_norm, float * out, void * q32a, void * q32b, unsigned short * q32meta, void * stream);

/*
 * Prefill of positions pos .. pos+T-1 of sequence seq (pos = the stored length, no gap) for slots layer0 ..
 * layer0+n_layers-1: stores the K/V rows (k, v [T][n_layers][4][256], dtype as mk_kv_append) and computes the causal
 * attention of the chunk's queries (q [n_layers][T][24][256], after RMSNorm/RoPE) over the store, out of the same
 * shape.  The chunk runs in pieces ending at 640-position bucket boundaries, each piece stored and then attended, so
 * its rows read the window of their bucket from the ring (MK_EXACT prefill, prefill_host.cu:606-615).  Each output
 * is a function of its position and the stored rows only: the result does not depend on how a prompt is split into
 * chunks (pk_attn8's exact form, prefill_attn.cuh:698-702).  Replaces pk_attn_prep's kv_store + attn (pk_attn8 /
 * pk_attn9 + combine) of mk_prefill.  Asynchronous on `stream`.
 */
int mk_kv_prefill(void * h, int seq, int layer0, int n_layers, int pos, int T, const void * k, const void * v, int dtype, const float * q,
                  float * out, void * stream);

/*
 * mk_kv_prefill on the raw projections with the whole attention block of a prefill layer: K before the k-norm / RoPE
 * (fp32), qg [n_layers][T][24][512] (query 256 | gate 256 per head), k_norm / q_norm [n_layers][256]; out gated, and
 * the optional q32 set [n_layers][T][192][16 | 4] as mk_kv_attend_gated (pk_attn_prep, attention, pk_attn_out:
 * prefill.cuh:986-1060).
 */
int mk_kv_prefill_prep(void * h, int seq, int layer0, int n_layers, int pos, int T, const float * k, const float * v, const float * k_norm,
                       const float * qg, const float * q_norm, float * out, void * q32a, void * q32b, unsigned short * q32meta,
                       void * stream);

/* Rewind sequence 0 / sequence seq to position pos: ring rows refilled from the main store (ring_rewind,
 * ck_pool.cu:285-296; k_ring_refill, qwen38_mk.cu:2485-2517).  mk_truncate / mk_rewind_to replace capi.cpp:572 / 601. */
int mk_truncate(void * h, int len);
int mk_rewind_to(void * h, int pos);
int mk_kv_rewind(void * h, int seq, int pos);

/* Bytes per KV token (all slots, both sides, values + scales), of the window rings, of the recurrent state (0: none in
 * this store) and of one checkpoint (0).  Replaces mk_kv_sizes, capi.cpp:675. */
void mk_kv_sizes(void * h, long long * per_token, long long * rings, long long * state, long long * checkpoint);

/* 64-bit digests of the KV state of sequence 0 / seq (the reference's layout restricted to the KV rows, engine.cu:1436-1514):
 * words [0x4d4b444701, n, 0, kvrc, ring_lo, n_layers, 4, 0], then per (slot, side, kv head, p < n) the main row's hash,
 * then per (slot, side, kv head, ring_lo <= p < n) the ring row's hash (0 for sides without a ring).  Returns the word
 * count (writes up to cap).  Replaces mk_state_digest, capi.cpp:635. */
int mk_state_digest(void * h, unsigned long long * out, int cap);
int mk_kv_state_digest(void * h, int seq, unsigned long long * out, int cap);

/* Copy n logical rows (positions p0 .. p0+n-1) of one (slot, side w, kv head g) to host memory: from the main store
 * (ring = 0; vals n * 32 * bits bytes) or the window ring (ring = 1; n * 256 bytes); scales n * 8 fp16.  Returns the
 * row bytes.  Test and park/unpark helper (host_store.cu:80-160 copies the same rows). */
int mk_kv_read_rows(void * h, int seq, int layer, int w, int g, int p0, int n, int ring, void * vals, unsigned short * scales);

/* Write n logical rows back into the store (the unpark half of host_store.cu:80-160's park/unpark copies): main-store
 * rows (ring = 0; vals n * 32 * bits bytes) or window-ring rows (ring = 1; n * 256 bytes, n <= ring rows), scales
 * n * 8 fp16, from host memory.  The sequence's stored length grows to cover them.  Returns 0. */
int mk_kv_write_rows(void * h, int seq, int layer, int w, int g, int p0, int n, int ring, const void * vals, const unsigned short * scales);

/* Window-ring snapshots for exact checkpoint reuse (the MK_EXACT ring copies of a checkpoint save / restore,
 * ck_pool.cu:39-42, 135-194, 268-296).  mk_kv_ring_snapshot copies every ring of sequence seq (with a header holding
 * the store layout and the sequence's position) to dst (host or device memory) and returns the byte count; dst NULL
 * or cap too small returns the count needed and copies nothing.  mk_kv_ring_restore puts a snapshot back and rewinds
 * the sequence to pos (<= the snapshot's position): ring rows the snapshot holds are restored bit for bit, older
 * window rows are refilled from the main rows as mk_kv_rewind does.  Both synchronise the device. */
long long mk_kv_ring_snapshot(void * h, int seq, void * dst, long long cap);
int mk_kv_ring_restore(void * h, int seq, int pos, const void * src, long long bytes);

/* Knobs: "max_blocks" caps the attention grid (0: one workgroup per work item); "occupancy" sets the decode
 * workgroups per CU for one-token calls on packed formats of at most 11 bits per K + V value: 0 (default) = three
 * when a launch has more work items than two per CU hold, else two; 2 or 3 = always that; "wide" (T >= 5): 1 = one
 * pass over K/V with 8-wave workgroups holding all 48 rows, 0 = two passes of 24 rows (the second pass's tiles found in
 * the same XCD's L2), 2 (default) = the faster of the two as measured, the two passes, on every format.  Results never
 * depend on any of them. */
int mk_kv_config(void * h, const char * key, long long value);

/* Kernel timing with HIP events on the launch stream (the reference's MK_PROFILE per-phase means, engine.cu:382-506).
 * enable = 1 resets and starts recording every attend call's attention and combine kernels (the query preparation
 * runs inside the attention kernel) and every append; 0 stops.
 * out[0..4): attend calls, then total milliseconds of attention, combine, append.  Returns the count written. */
int mk_kv_profile(void * h, int enable, double * out, int cap);

/* Host-only geometry and grammar helpers (no GPU needed). */
int mk_kv_window_start(int L, int win);  /* kv_ws, qwen38_mk.cu:2118-2126 */
int mk_kv_ring_rows(int win);            /* kvrc, loader.cu:1479-1486 */
int mk_kv_cap_T(int n, int T);           /* att_cap_T, mk_shared.cuh:288-291 */
/* Parse an MK_KV spec for n_layers slots: out[0..n) K bits, [n..2n) V bits, [2n..3n) K rotated, [3n..4n) V rotated.
 * Returns 0, or -1 with mk_last_error (loader.cu:1329-1365's messages). */
int mk_kv_parse_spec(const char * kv_spec, int n_layers, int * out);

#ifdef __cplusplus
}
#endif

#endif
