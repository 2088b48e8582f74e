/*
 * strict_topk.h -- C ABI of libstrict_topk_hip.so, the gfx950 HIP kernels of
 * the speculative block-sparse Top-K decode path.
 *
 * Each entry point replaces one host function of the reference's Python
 * package (6Mikao9/strict-topk-overlap, files under strict_topk/); the
 * citation above each declaration names it.  The reference binds no C ABI:
 * its host functions launch Triton kernels.  The binding that takes the
 * place of those launches is strict_topk/_lib.py (ctypes) in this repository.
 *
 * Conventions shared by every entry point
 *   - Pointers are device addresses; every buffer is contiguous, row-major.
 *     q[Hq,D]; k,v[Hkv,N,B,D] (Hq % Hkv == 0, query head h reads KV head
 *     h / (Hq/Hkv)); lo,hi[Hkv,N,D] float32; ID rows [Hq,S]; states
 *     m,l[Hq,S] and u[Hq,S,D] float32; outputs float32.
 *   - dtype codes: STK_F32, STK_F16, STK_BF16 (elements of q, k, v);
 *     ID codes: STK_I32, STK_I64.  Boolean arrays are one byte per entry
 *     (torch.bool layout).
 *   - `stream` is a hipStream_t.  Every call only enqueues work on it: no
 *     allocation, no host synchronisation, no copy to the host, so calls can
 *     be captured into a HIP graph and issued on concurrent streams.
 *   - Bounds lo/hi (and lo/hi pages) are float32, or, where an entry point
 *     takes `bounds_dtype`, optionally stored in the keys' own 16-bit type
 *     (bounds_dtype = dtype): the min / max of 16-bit keys are 16-bit values,
 *     so that storage is exact, scores and selections are the same bits, and
 *     the scorer reads half the bytes.  bounds_dtype = STK_F32 is the
 *     reference's layout.
 *   - Scratch memory beyond inputs and outputs is the caller's `workspace`
 *     of at least the size the matching *_workspace_bytes() returns.
 *   - ID values are not validated on the device; an ID outside [0, N)
 *     contributes an empty state (-inf, 0, 0) and never reads memory.
 *   - Return value: STK_OK, STK_EINVAL (bad argument; nothing launched) or
 *     STK_EHIP (launch error).  stk_last_error() gives the calling thread's
 *     last message.
 */
#ifndef STRICT_TOPK_H
#define STRICT_TOPK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { STK_OK = 0, STK_EINVAL = -1, STK_EHIP = -2 };
enum { STK_F32 = 0, STK_F16 = 1, STK_BF16 = 2 };
enum { STK_I32 = 0, STK_I64 = 1 };
enum { STK_SAVED = 0, STK_HYBRID = 1, STK_COMPACT = 2 };

const char* stk_last_error(void);
int stk_abi_version(void);

/* ---------------------------------------------------------- selection */

/* strict_topk/selector.py:23-38 block_scores (and gqa.py:15-26 scoring):
 * scores[h,n] = sum_d q_d * (q_d >= 0 ? hi : lo)[h/G, n, d], evaluated in
 * float64 in a fixed order, stored as float32. */
int stk_block_scores(const void* q, int q_dtype, const void* lo, const void* hi,
                     int bounds_dtype, int hq, int hkv, int n, int d, float* scores,
                     void* stream);

size_t stk_select_workspace_bytes(int hq, int hkv, int n, int d, int topk);

/* strict_topk/selector.py:41-43 select_blocks and gqa.py:145-161
 * select_blocks (score + torch.topk(sorted=False)): ids[h, 0..topk) are the
 * topk highest-scoring blocks, ties toward the lower block index, in
 * ascending block order.  `scores` may be NULL. */
int stk_select_blocks(const void* q, int q_dtype, const void* lo, const void* hi,
                      int bounds_dtype, int hq, int hkv, int n, int d, int topk, float* scores,
                      int32_t* ids, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------- states and merge */

/* strict_topk/kernels.py:425-434 block_partials and gqa.py:128-137 partials:
 * per (query head, slot) m = max logit, l = sum exp(logit - m),
 * u = sum exp(logit - m) V, logits = q.k / sqrt(D).  `active` (may be NULL)
 * is [Hq] (active_kind 1) or [Hq,S] (active_kind 2); inactive slots get
 * (-inf, 0, 0). */
int stk_block_partials(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                       int n, int b, int d, const void* ids, int id_dtype, int s,
                       const uint8_t* active, int active_kind, float* m, float* l, float* u,
                       void* stream);

/* strict_topk/kernels.py:437-442 merge_partials: LSE merge of S states per
 * head, optional include mask [H,S], out = sum e^(m-M) u / max(z, 1e-30). */
int stk_merge_partials(const float* m, const float* l, const float* u, const uint8_t* include,
                       int h, int s, int d, float* out, void* stream);

size_t stk_exact_workspace_bytes(int hq, int s, int d);

/* strict_topk/kernels.py:445-447 exact_attention and gqa.py:140-142 exact. */
int stk_exact_attention(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                        int n, int b, int d, const void* ids, int id_dtype, int s, float* out,
                        void* workspace, size_t workspace_bytes, void* stream);

/* strict_topk/kernels.py:450-501 speculate (saved / hybrid / compact).
 * saved: m,l,u[Hq,s].  hybrid: also high[Hq,s], low_m/low_l[Hq], low_u and
 * low_abs[Hq,D].  compact (capacity C from kernels.py:485): m,l,u[Hq,C],
 * retained_ids[Hq,C] (pred_dtype, rank order, -1 padded), overflow[Hq],
 * mass_m/mass_l[Hq,s] required.  Unused outputs may be NULL. */
int stk_speculate(const void* q, const void* k, const void* v, int dtype, int hq, int hkv, int n,
                  int b, int d, const void* pred, int pred_dtype, int s, int mode, float tau,
                  int capacity, float* m, float* l, float* u, uint8_t* high, float* low_m,
                  float* low_l, float* low_u, float* low_abs, void* retained_ids,
                  uint8_t* overflow, float* mass_m, float* mass_l, void* stream);

/* strict_topk/kernels.py:553-560 touch_kv: per (head, slot, 1024-element
 * tile) sum of K + V of the predicted block, out[H,S,ceil(B*D/1024)]. */
int stk_touch_kv(const void* k, const void* v, int dtype, int h, int n, int b, int d,
                 const void* pred, int pred_dtype, int s, float* out, void* stream);

/* ------------------------------------------------------------- repairs */

/* strict_topk/kernels.py:223-247 _fallback (as launched by kernels.py:548
 * and signed_repair.py:231): strict online softmax over the selected set on
 * heads whose flag is set. */
int stk_fallback(const void* q, const void* k, const void* v, int dtype, int hq, int hkv, int n,
                 int b, int d, const void* selected, int sel_dtype, int sa, const uint8_t* flags,
                 float* out, void* stream);

size_t stk_repair_workspace_bytes(int hq, int sa, int sp, int sc, int d, int mode);

/* strict_topk/kernels.py:504-550 repair (split path: membership, miss
 * states, saved or hybrid merge with guards, fallback).  (pm,pl,pu) is the
 * prediction state of width sc; high/low_* are required for hybrid and
 * compact, retained_ids for compact. */
int stk_repair(const void* q, const void* k, const void* v, int dtype, int hq, int hkv, int n,
               int b, int d, const void* selected, int sel_dtype, int sa, const void* predicted,
               int pred_dtype, int sp, int mode, int sc, const float* pm, const float* pl,
               const float* pu, const uint8_t* high, const float* low_m, const float* low_l,
               const float* low_u, const float* low_abs, const void* retained_ids,
               float min_remaining, float cancellation_tol, float* out, uint8_t* fallback,
               float* remaining, void* workspace, size_t workspace_bytes, void* stream);

/* strict_topk/fused.py:176-220 repair_fused: the whole repair in one
 * workgroup per head, with the extra-mass budget max_extra_mass
 * (approximate/extra_mass_bound [Hq] required when it is > 0). */
int stk_repair_fused(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                     int n, int b, int d, const void* selected, int sel_dtype, int sa,
                     const void* predicted, int pred_dtype, int sp, int mode, int sc,
                     const float* pm, const float* pl, const float* pu, const uint8_t* high,
                     const float* low_m, const float* low_l, const float* low_u,
                     const float* low_abs, const void* retained_ids, const float* mass_m,
                     const float* mass_l, float min_remaining, float cancellation_tol,
                     float max_extra_mass, float* out, uint8_t* fallback, float* remaining,
                     uint8_t* approximate, float* extra_mass_bound, void* stream);

size_t stk_gqa_repair_workspace_bytes(int hq, int sa, int d);

/* strict_topk/gqa.py:164-193 repair_saved (union_mode 0) and repair_union
 * (union_mode 1) for native GQA. */
int stk_gqa_repair(const void* q, const void* k, const void* v, int dtype, int hq, int hkv, int n,
                   int b, int d, const void* selected, int sel_dtype, int sa,
                   const void* predicted, int pred_dtype, int sp, const float* pm,
                   const float* pl, const float* pu, int union_mode, float* out,
                   void* workspace, size_t workspace_bytes, void* stream);

/* strict_topk/gqa_light.py:63-77 repair_saved_light: hits merged from the
 * saved states, misses streamed with the online softmax, one launch. */
int stk_repair_light(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                     int n, int b, int d, const void* selected, int sel_dtype, int sa,
                     const void* predicted, int pred_dtype, int sp, const float* pm,
                     const float* pl, const float* pu, float* out, void* stream);

size_t stk_signed_workspace_bytes(int hq, int sa, int sp, int sc, int d, int mode);

/* strict_topk/signed_repair.py:175-232 repair_signed (fused 0: schedule,
 * signed partials, guarded merge, separate fallback) and
 * strict_topk/signed_fused.py:148-193 repair_signed_fused (fused 1:
 * schedule, signed corrections, finalize with inline fallback).  queue is
 * [Hq, sa + sp] (hybrid/compact) or [Hq, sa] (saved) of queue_dtype;
 * positive_jobs/total_jobs are [Hq] int32. */
int stk_repair_signed(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                      int n, int b, int d, const void* selected, int sel_dtype, int sa,
                      const void* predicted, int pred_dtype, int sp, int mode, int sc,
                      const float* pm, const float* pl, const float* pu, const uint8_t* high,
                      const float* low_m, const float* low_l, const float* low_u,
                      const float* low_abs, const void* retained_ids, const float* mass_m,
                      const float* mass_l, float min_remaining, float cancellation_tol,
                      float max_extra_mass, int fused, void* queue, int queue_dtype,
                      int32_t* positive_jobs, int32_t* total_jobs, float* out, uint8_t* fallback,
                      float* remaining, uint8_t* approximate, float* extra_mass_bound,
                      void* workspace, size_t workspace_bytes, void* stream);

/* --------------------------------------------------------- hierarchical */

size_t stk_hier_exact_workspace_bytes(int hq, int s, int d);

/* strict_topk/gqa_hierarchical.py:111-112 exact: per-block states, level-1
 * merge of 32 positions, final LSE merge. */
int stk_hier_exact(const void* q, const void* k, const void* v, int dtype, int hq, int hkv, int n,
                   int b, int d, const void* selected, int sel_dtype, int sa, float* out,
                   void* workspace, size_t workspace_bytes, void* stream);

size_t stk_hier_repair_workspace_bytes(int hq, int sa, int d, int shared);

/* strict_topk/gqa_hierarchical.py:115-144 repair_saved (shared 0) and
 * repair_saved_shared (shared 1: row 0's slot table serves every head). */
int stk_hier_repair(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                    int n, int b, int d, const void* selected, int sel_dtype, int sa,
                    const void* predicted, int pred_dtype, int sp, const float* pm,
                    const float* pl, const float* pu, int shared, float* out, void* workspace,
                    size_t workspace_bytes, void* stream);

/* ---------------------------------------------- shared-selection indexer */

size_t stk_indexer_workspace_bytes(int n);

/* The QSA indexer formula of benchmarks/selector_window.py:126-142
 * (_indexer_scores / qsa_reference_scores): scores[n] = sum_h relu(iq_h .
 * ik_n) / sqrt(D) over iq[H,D], ik[N,D] (fp32 / fp16 / bf16), H * D <= 4096,
 * evaluated in FP64 in a fixed order, stored as float32. */
int stk_indexer_scores(const void* iq, const void* ik, int dtype, int h, int n, int d,
                       float* scores, void* workspace, size_t workspace_bytes, void* stream);

/* The shared selector of benchmarks/selector_window.py:76-84 (indexer scores,
 * scores.topk(topk, sorted=False), the row expanded to every query head):
 * ids[rows, topk] int32, every row the same topk highest-scoring keys, ties
 * toward the lower index, ascending.  `scores` may be NULL. */
int stk_indexer_select(const void* iq, const void* ik, int dtype, int h, int n, int d, int topk,
                       int rows, float* scores, int32_t* ids, void* workspace,
                       size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------ block bounds */

/* Block metadata of the bound scorer: lo/hi[Hkv, N, D] FP32 = per-block,
 * per-dim minimum / maximum of k[Hkv, N, B, D] over the B tokens, as the
 * reference harness builds them with k.amin(dim=2).float() / k.amax(dim=2)
 * (benchmarks/critical_path.py:186, benchmarks/run_benchmark.py:43).  NaN
 * keys give NaN bounds, as torch does.  k: fp32 / fp16 / bf16; bounds_dtype:
 * STK_F32, or the 16-bit dtype of k (exact, half the bytes). */
int stk_block_bounds(const void* k, int dtype, int hkv, int n, int b, int d, void* lo, void* hi,
                     int bounds_dtype, void* stream);

/* Decode append: the token k_new[Hkv, D] lands at position `pos` of block
 * `block`; pos 0 starts the block's bounds over, otherwise they widen.  The
 * reference has no counterpart (its harness rebuilds lo/hi outside timing);
 * this is the per-token update a decode loop needs. */
int stk_bounds_append(const void* k_new, int dtype, int hkv, int n, int d, int block, int pos,
                      void* lo, void* hi, int bounds_dtype, void* stream);

/* ------------------------------------------------------- fused decode step */

size_t stk_step_workspace_bytes(int hq, int hkv, int n, int d, int topk);

/* 1 when stk_speculative_step supports the shape (alignment aside). */
int stk_step_supported(int dtype, int hq, int hkv, int n, int b, int d, int topk, int sp,
                       int pred_dtype);

/* The full speculative decode step of benchmarks/run_benchmark.py:99-118
 * (overlap_run: gqa.select_blocks || gqa.partials on the predicted blocks,
 * then gqa_light.repair_saved_light / gqa.repair_saved, or gqa.repair_union
 * with union_mode 1) on one stream: one workgroup per query head where
 * stk_step_small_supported says so, else one launch where
 * stk_step1_supported says so, otherwise two launches (a grid whose workgroups either score
 * blocks or compute the predicted blocks' states, then one workgroup per
 * query head doing the exact top-K and the repair).  Outputs:
 * selected[Hq,topk] int32 (ascending IDs, as stk_select_blocks), the
 * prediction state m,l[Hq,sp], u[Hq,sp,D] (as stk_block_partials) and
 * out[Hq,D].  bf16/fp16 only, int32 predicted IDs, D in {64, 128, 256}. */
int stk_speculative_step(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                         int n, int b, int d, const void* lo, const void* hi, int bounds_dtype,
                         int topk, const void* predicted, int pred_dtype, int sp,
                         int union_mode, int32_t* selected, float* m, float* l, float* u,
                         float* out, void* workspace, size_t workspace_bytes, void* stream);

/* 1 when stk_speculative_step (and stk_speculative_step_noalloc) run the
 * shape as ONE launch: bf16/fp16, B = 32, D in {64, 128}, at most four query
 * heads per KV head, SP * D <= 8192, Hq * (ceil(N / 64) + SP) < 16384, within
 * the shapes of stk_step_supported.  The one launch is a grid whose workgroups score
 * blocks, compute the predicted blocks' states, or (the last Hq workgroups)
 * wait for their head's scores, run the top-K and the repair while the
 * states still stream, then wait for the states and merge; the roles hand
 * over through flags the library keeps in static device memory, one slot per
 * stream (64 slots per device; with every slot taken the step runs as two
 * launches).  A graph captured on a stream keeps that stream's slot: it must
 * not be replayed on another stream while the capturing stream runs the step
 * at the same time (capture on a stream of its own).  Results are the two
 * launches' results, bit for bit.  No
 * reference counterpart beyond the step it computes
 * (benchmarks/run_benchmark.py:99-118). */
int stk_step1_supported(int dtype, int hq, int hkv, int n, int b, int d, int topk, int sp,
                        int pred_dtype);

/* 1 when stk_speculative_step (and stk_speculative_step_noalloc) run the
 * shape in one workgroup per query head, with no hand-off between
 * workgroups: bf16/fp16, B = 32, D in {64, 128}, N <= 128, TOPK and SP in
 * [1, 16], int32 predicted IDs, bounds FP32 or of the K/V type (16-byte
 * aligned pointers assumed; others take the paths above).  Such a head's
 * bounds, then its misses' tiles, are two dependent memory round trips of
 * its own workgroup; its predicted tiles travel beside them.  The selected
 * IDs are those of every other path (the same FP64 scores); the states and
 * the output equal the oracle's within the step's tolerance, and since a
 * miss is merged as two 16-token halves their bits may differ from the
 * other paths'.  No reference counterpart beyond the step it computes
 * (benchmarks/run_benchmark.py:99-118). */
int stk_step_small_supported(int dtype, int hq, int hkv, int n, int b, int d, int topk, int sp,
                             int pred_dtype, int bounds_dtype);

/* Slots of the current device whose one-launch step ever timed out waiting
 * for a flag (each wait gives up after 20 ms, so every launch ends, and the
 * head that waited gets a NaN output and IDs of -1); 0 in any correct run.  A host-side query that copies from the device (it waits for
 * the device); for tests. */
int stk_step1_timeouts(void);

/* Test hook, no reference counterpart: sets the one-launch step's longest
 * wait (spin_ticks of the 100 MHz counter; 2000000 by default) and, with
 * drop_flags 1, makes its producers publish no flag, so that every wait times
 * out and the kernel still ends.  A tail whose wait timed out writes NaN
 * outputs and IDs of -1 for its head.  Clears the time-out counters of the
 * current device (a synchronous copy).  For failure-handling tests only. */
int stk_step1_test_hook(unsigned long long spin_ticks, int drop_flags);

/* Allocation-free variant of stk_speculative_step.  It has no counterpart in
 * the reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, results and shape support as stk_speculative_step, without the
 * workspace: the score keys live in a fixed array of device memory inside the
 * library, one per GPU (4 MiB, held until the process ends), so Hq * N may
 * not exceed stk_step_noalloc_max_keys() (524288); larger shapes return
 * STK_EINVAL.  Shapes of stk_step1_supported run as one launch, with the
 * flags in the library's per-stream slots.  The call allocates nothing, not
 * even on its first use on a device (it then only looks up the array's and
 * the slots' addresses; that first use must not be under stream capture, see
 * stk_step_prepare).  Calls on one GPU share the array: calls that overlap in
 * time on one GPU (on concurrent streams) race and must be ordered by the
 * caller. */
size_t stk_step_noalloc_max_keys(void);

/* Looks up, on the current device, the device memory the fused step keeps in
 * the library (the allocation-free step's array and the one-launch step's
 * flag slots).  The step entry points do this on a device's first call, and
 * refuse to (STK_EINVAL) when that first call is made under stream capture:
 * a caller that captures before any eager call makes this call first,
 * outside the capture.  It has no reference counterpart. */
int stk_step_prepare(void);

int stk_speculative_step_noalloc(const void* q, const void* k, const void* v, int dtype, int hq,
                                 int hkv, int n, int b, int d, const void* lo, const void* hi,
                                 int bounds_dtype, int topk, const void* predicted,
                                 int pred_dtype, int sp, int union_mode, int32_t* selected,
                                 float* m, float* l, float* u, float* out, void* stream);

/* The two launches of stk_speculative_step separately.  stk_step_front
 * (select || speculate) writes the prediction state and the score keys into
 * `workspace`; stk_step_tail (top-K + repair) reads them from the same
 * workspace and writes `selected` and `out`. */
int stk_step_front(const void* q, const void* k, const void* v, int dtype, int hq, int hkv, int n,
                   int b, int d, const void* lo, const void* hi, int bounds_dtype, int topk,
                   const void* predicted, int pred_dtype, int sp, float* m, float* l, float* u,
                   void* workspace, size_t workspace_bytes, void* stream);

int stk_step_tail(const void* q, const void* k, const void* v, int dtype, int hq, int hkv, int n,
                  int b, int d, int topk, const void* predicted, int pred_dtype, int sp,
                  int union_mode, const float* m, const float* l, const float* u,
                  int32_t* selected, float* out, void* workspace, size_t workspace_bytes,
                  void* stream);

/* The signed speculative decode step: gqa.select_blocks (strict_topk/gqa.py:145-161)
 * || kernels.speculate(mode, mass_threshold, keep_mass=True)
 * (strict_topk/kernels.py:450-477, _group :94-117), then
 * signed_fused.repair_signed_fused (strict_topk/signed_fused.py:148-193:
 * _schedule signed_repair.py:18-82, _corrections :30-67, _finalize :70-145),
 * in two launches on one stream (the scoring and state grid of
 * stk_speculative_step's two-launch form, then one workgroup per query head doing the top-K, the grouping, the signed
 * corrections, the guarded merge and the strict fallback).  hybrid 1: hybrid
 * prediction, 0: saved.  Outputs: selected[Hq,topk] int32 ascending, the
 * prediction state m,l[Hq,sp], u[Hq,sp,D], out[Hq,D], fallback[Hq] and
 * approx[Hq] as bytes 0/1, remaining[Hq], extra[Hq], positive and total job
 * counts [Hq] int32; approx and extra may be null when max_extra_mass == 0.
 * Supported shapes are those of stk_step_supported; the workspace is
 * stk_step_workspace_bytes. */
int stk_signed_step(const void* q, const void* k, const void* v, int dtype, int hq, int hkv,
                    int n, int b, int d, const void* lo, const void* hi, int bounds_dtype,
                    int topk,
                    const void* predicted, int pred_dtype, int sp, int hybrid,
                    float mass_threshold, float min_remaining, float cancellation_tol,
                    float max_extra_mass, int32_t* selected, float* m, float* l, float* u,
                    float* out, uint8_t* fallback, float* remaining, uint8_t* approx,
                    float* extra, int32_t* positive, int32_t* total, void* workspace,
                    size_t workspace_bytes, void* stream);

/* ---- Paged, ragged KV and batched steps.
 * Replaces the page-table indirection of strict_topk/flashinfer_backend.py:35-40
 * (_pages: page = block + kv_head * N over k.view(hkv * n, b, 1, d), one
 * request per FlashInfer call) with a native wire format shared by a whole
 * batch of R requests:
 *   k_pages, v_pages [pages, B, D]   one page = one KV head's block of B tokens
 *   lo_pages, hi_pages [pages, D]    per-dim key min / max of the page, FP32
 *                                    or the pages' 16-bit type (bounds_dtype)
 *                                    (stk_block_bounds on the pool as
 *                                    hkv = 1, n = pages)
 *   block_table [R, Hkv, nb] int32   page of logical block j of (request r,
 *                                    KV head kvh), valid for j < nblocks[r]
 *   nblocks [R] int32                blocks per request (device memory)
 *   ntokens [R] int32 or null        tokens per request (device memory): token
 *                                    t of block j holds data when
 *                                    j * B + t < ntokens[r], so a request's
 *                                    last block may be partly filled (its
 *                                    other tokens get no weight, whatever the
 *                                    page holds); null: every block is full
 *   q [R, Hq, D]; predicted [R, Hq, sp] int32 logical block IDs.
 * Per request the results are those of stk_speculative_step /
 * stk_signed_step on the request's blocks gathered from the pool, except
 * that a request with fewer blocks than topk selects all of them (the rest
 * of its ID row is -1).  A table entry outside [0, pages) is an invalid
 * page: its block scores lowest and has the empty state, and nothing is
 * read from it.  sp may be 0 (predicted, m, l, u may then be null): the step
 * is then the serial path, the exact attention over the selected blocks.
 * Outputs are laid out [R, Hq, ...] like q.  Shapes: those of
 * stk_step_supported with n = nb and topk, sp <= 256. */
size_t stk_paged_workspace_bytes(int requests, int hq, int nb);

/* One decode token per request into the pool: k_new, v_new [R, Hkv, D] go to
 * token position positions[r] (block pos / B, offset pos % B) of the page
 * block_table[r, kvh, pos / B]; that page's lo/hi are widened by the new key
 * (offset 0 starts them over, as stk_bounds_append does for the dense layout)
 * and nblocks[r] becomes pos / B + 1, ntokens[r] (when not null) pos + 1.
 * A position outside [0, nb * B) writes nothing; an invalid page writes
 * nothing for its KV head, and the counts change only when the block has a
 * valid page for every KV head.  The reference has no decode append (its
 * harness builds the bounds once, benchmarks/critical_path.py:186); this is
 * the paged form of stk_bounds_append plus the K/V write. */
int stk_paged_append(const void* k_new, const void* v_new, int dtype, int requests, int hkv,
                     int nb, int b, int d, int pages, void* k_pages, void* v_pages,
                     void* lo_pages, void* hi_pages, int bounds_dtype,
                     const int32_t* block_table,
                     int32_t* nblocks, int32_t* ntokens, const int32_t* positions,
                     void* stream);

/* stk_speculative_step over a paged batch (union_mode: repair_union). */
int stk_paged_step(const void* q, const void* k_pages, const void* v_pages, int dtype,
                   int requests, int hq, int hkv, int nb, int b, int d, int pages,
                   const void* lo_pages, const void* hi_pages, int bounds_dtype,
                   const int32_t* block_table,
                   const int32_t* nblocks, const int32_t* ntokens, int topk,
                   const int32_t* predicted, int sp, int union_mode, int32_t* selected, float* m,
                   float* l, float* u, float* out, void* workspace, size_t workspace_bytes,
                   void* stream);

/* stk_signed_step over a paged batch. */
int stk_paged_signed_step(const void* q, const void* k_pages, const void* v_pages, int dtype,
                          int requests, int hq, int hkv, int nb, int b, int d, int pages,
                          const void* lo_pages, const void* hi_pages, int bounds_dtype,
                          const int32_t* block_table, const int32_t* nblocks,
                          const int32_t* ntokens, int topk, const int32_t* predicted, int sp,
                          int hybrid, float mass_threshold,
                          float min_remaining, float cancellation_tol, float max_extra_mass,
                          int32_t* selected, float* m, float* l, float* u, float* out,
                          uint8_t* fallback, float* remaining, uint8_t* approx, float* extra,
                          int32_t* positive, int32_t* total, void* workspace,
                          size_t workspace_bytes, void* stream);

/* ---- Host-backed cache (docs/hisparse_integration.md:11-27: a pinned host
 * KV pool, a device working set per request, swap-in of the selected blocks
 * that are not resident, speculation on the resident predicted blocks
 * P n R only).  Layout, all device memory unless said otherwise:
 *   host_k, host_v [host_pages, B, D]  pinned host memory the GPU reads in
 *                                      place (hipHostMalloc)
 *   lo_pages, hi_pages [host_pages, D] every block's bounds (bounds_dtype)
 *   host_table [R, Hkv, nb] int32      host page of logical block j
 *   k_slots, v_slots [R * Hkv * C, B, D]  device slots; group r * Hkv + kvh
 *                                      owns slots [g * C, g * C + C)
 *   table [R, Hkv, nb] int32           device slot of block j, or -1
 *   slot_block [R * Hkv * C] int32     block a slot holds, or -1
 *   slot_stamp [R * Hkv * C] int32     step of a slot's last use
 *   clock [1] int32                    step counter (advanced by each step)
 *   nblocks, ntokens [R]               as in the paged format
 * One step (five launches): scores of every block || prediction states of
 * the resident predicted blocks (a non-resident one has the empty state);
 * the top-K; swap-in per (request, KV head): selected blocks without a slot
 * take the least recently used slots not needed this step (free ones first)
 * and are copied from the host pool by a copy kernel, *h2d_bytes grows by the
 * bytes copied;
 * then the strict repair from the slots.  Outputs as stk_paged_step, over
 * the request's selected set A; sp = 0 (predicted, m, l, u may be null) is
 * the serial path: select, swap-in, then the exact attention over A.  Needs G * topk <= C <= 1024, nb <= 8192,
 * bf16 / fp16.  The reference has no such kernels (it describes the design
 * for SGLang's HiSparse); this is its native form here. */
size_t stk_cache_workspace_bytes(int requests, int hq, int hkv, int nb);

int stk_cache_step(const void* q, int dtype, int requests, int hq, int hkv, int nb, int b, int d,
                   void* k_slots, void* v_slots, int slots_per_group, const void* host_k,
                   const void* host_v, int host_pages, const void* lo_pages,
                   const void* hi_pages, int bounds_dtype, const int32_t* host_table,
                   int32_t* table, int32_t* slot_block, int32_t* slot_stamp, int32_t* clock,
                   const int32_t* nblocks, const int32_t* ntokens, int topk,
                   const int32_t* predicted, int sp, int32_t* selected, float* m, float* l,
                   float* u, float* out, unsigned long long* h2d_bytes, void* workspace,
                   size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* STRICT_TOPK_H */
