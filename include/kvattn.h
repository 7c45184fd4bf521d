/* kvattn.h -- C ABI of the MI355X (gfx950) decode-phase KV-cache attention library.
 *
 * Drop-in for the attention call inside a GPT-2 decode step: the same q / K-cache /
 * V-cache / out pointer layouts as the reference engine, the same [NH, maxT, hs] cache
 * slot per (batch, head), a device-resident current length (so captured graphs stay
 * valid while the length grows), and the FP32 / BF16 / INT8 / FP8-E4M3 KV switch, here a
 * run-time argument instead of a compile-time macro.
 *
 * Layouts (reference names; element type below):
 *   qkv       [B][3][NH][hs]             Q, K, V of the current token
 *   kv_cache  [2][B][NH][maxT][hs]       K block then V block; K(b,h,j) at
 *                                        ((b*NH+h)*maxT + j)*hs, V adds B*NH*maxT*hs
 *   kv_scale  [2][B][NH][maxT] float     per-row scales, 8-bit caches only
 *   out       [B][NH][hs]
 *   part_out  [B][NH][S][hs] float, part_max / part_lse [B][NH][S] float
 * Element types: kv_dtype F32 -> qkv, kv_cache, out are float.  BF16 -> bfloat16.
 * INT8 / FP8_E4M3 -> kv_cache holds one byte per element, qkv and out are bfloat16.
 *
 * Lengths: the number of attended positions of sequence b is cur_len + 1 where cur_len
 * is read ON THE DEVICE when the kernels run: from d_cur_len[0] for every sequence, or
 * from d_cur_len[b] when lens_per_seq != 0 (ragged batches).  d_cur_len == NULL means
 * the library's own device-resident length, see kvattn_cur_len_symbol().  Device lengths
 * are clamped into [0, maxT-1]; the host never reads them.
 *
 * Every entry point only enqueues work on `stream` (a hipStream_t; NULL = the null
 * stream), returns a kvattn_status and never exits the process.  All except the
 * cooperative strategy are legal inside hipStreamBeginCapture / hipStreamEndCapture.
 * Only hs == 64 is supported (one 64-lane wavefront spans one head row).
 */
#ifndef KVATTN_H
#define KVATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum kvattn_status {
    KVATTN_OK = 0,
    KVATTN_ERR_NULL_POINTER = 1,    /* a required pointer is NULL */
    KVATTN_ERR_MISALIGNED = 2,      /* qkv / kv_cache / out / workspace not 16-byte aligned */
    KVATTN_ERR_HEAD_DIM = 3,        /* hs != 64 */
    KVATTN_ERR_SHAPE = 4,           /* B, NH or maxT < 1, or a size that overflows */
    KVATTN_ERR_DTYPE = 5,           /* unknown kv_dtype, or kv_scale missing for 8-bit */
    KVATTN_ERR_STRATEGY = 6,        /* unknown strategy */
    KVATTN_ERR_WORKSPACE = 7,       /* workspace missing or smaller than required */
    KVATTN_ERR_SPLIT = 8,           /* S or seg_rows out of range */
    KVATTN_ERR_COOP_TOO_LARGE = 9,  /* cooperative grid exceeds co-resident capacity */
    KVATTN_ERR_LDS = 10,            /* fused_single scores for maxT do not fit in LDS */
    KVATTN_ERR_CAPTURE = 11,        /* cooperative launch requested inside stream capture */
    KVATTN_ERR_LENGTH = 12,         /* host length hint outside [0, maxT-1] */
    KVATTN_ERR_HIP = 13,            /* a HIP runtime call failed; see kvattn_last_hip_error */
    KVATTN_ERR_GRID_TOO_LARGE = 14, /* explicit SPLIT_DESIGNATED grid exceeds what the GPU holds
                                       at once (its mergers wait for their producers) */
    KVATTN_ERR_MERGE_TIMEOUT = 15   /* kvattn_workspace_status: a designated merger stopped
                                       waiting for its producers (and computed their segments
                                       itself), or a cooperative merger stopped waiting at the
                                       grid barrier (and wrote NaN) */
} kvattn_status;

typedef enum kvattn_dtype {
    KVATTN_KV_F32 = 0,       /* reference ENABLE_FP32 build (Makefile:78-79) */
    KVATTN_KV_BF16 = 1,      /* reference default BF16 build (Makefile:88-89) */
    KVATTN_KV_INT8 = 2,      /* reference USE_KV_W8 + USE_INT8 (Makefile:80-82,100-106) */
    KVATTN_KV_FP8_E4M3 = 3   /* reference USE_KV_W8 + USE_FP8 (Makefile:83-85,100-106) */
} kvattn_dtype;

typedef enum kvattn_strategy {
    KVATTN_AUTO = 0,                /* fused_single for short contexts, else a split plan
                                       chosen from len_hint, the shape and the cache type:
                                       the designated merger while its grid is small, one
                                       segment per (b,h) for many short heads, split +
                                       merge kernels once the call is bandwidth bound */
    KVATTN_FUSED_SINGLE = 1,        /* one workgroup per (b,h), scores staged in LDS */
    KVATTN_SPLIT_MERGE = 2,         /* flash-decoding: split kernel + merge kernel */
    KVATTN_SINGLE_LAUNCH_COOP = 3,  /* split + grid barrier + merge, cooperative launch */
    KVATTN_SINGLE_LAUNCH_GRAPH = 4, /* split + merge pair replayed as one hipGraph launch */
    KVATTN_SPLIT_LASTBLOCK = 5,     /* split kernel whose last finishing segment of each
                                       (b,h) merges: one ordinary launch, capturable */
    KVATTN_SPLIT_DESIGNATED = 6     /* split kernel in which segment 0 of each (b,h) merges:
                                       the other segments publish tagged partials and finish,
                                       segment 0 polls for them; one ordinary launch,
                                       capturable; at most 64 segments per (b,h).  AUTO's
                                       choice for latency-bound calls (with a length hint:
                                       grids of up to 768 workgroups, 1024 for up to 64
                                       heads with long segments, and 64 MiB of cache). */
} kvattn_strategy;

/* Human-readable text of a status code. */
const char* kvattn_strerror(int status);

/* The hipError_t of the most recent failing HIP call on this thread (0 if none). */
int kvattn_last_hip_error(void);

/* Device address of the library's device-resident length for the current device.
 * Replaces cudaGetSymbolAddress(&d_cur_len_ptr, g_cur_len)
 * (inference_gpt2_opt.cu:252-254; g_cur_len at Inference_gpt2/attention_kvcache.cuh:35-40). */
int kvattn_cur_len_symbol(int** d_cur_len);

/* Blocking write of the library's device-resident length.
 * Replaces cudaMemcpyToSymbol(g_cur_len, &cur_len, sizeof(int))
 * (inference_gpt2_opt.cu:409,548). */
int kvattn_set_cur_len(int cur_len);

/* Enqueue the write of cur_len into *d_cur_len (NULL: the library's own device length) on
 * `stream`, without a host synchronisation; capturable.  Replaces the per-token
 * cudaMemcpyToSymbol(g_cur_len, ...) before each graph replay (inference_gpt2_opt.cu:548),
 * which blocks the host until the copy is done. */
int kvattn_set_cur_len_async(int* d_cur_len, int cur_len, void* stream);

/* Append the current token's K and V (from qkv) into column cur_len of every (b,h) slot.
 * F32/BF16 copy the elements; INT8/FP8 quantise each 64-element row with
 * scale = amax/127 (INT8) or amax/448 (FP8), store the codes and the FP32 scale.
 * Replaces kv_cache_write_kernel (Inference_gpt2/attention_kvcache.cuh:46-64) and
 * kv_cache_write_kernel_w8 (Inference_gpt2/attention_kvcache_w8.cuh:115-155), launched at
 * inference_gpt2_opt.cu:302-303 and :329.  kv_scale must be NULL for F32/BF16. */
int kvattn_cache_write(void* kv_cache, float* kv_scale, const void* qkv,
                       int B, int NH, int hs, int maxT,
                       const int* d_cur_len, int lens_per_seq,
                       int kv_dtype, void* stream);

/* kvattn_cache_write with one length for the whole batch (lens_per_seq = 0): the append
 * with exactly the arguments of the reference's launch (kv_cache_write_kernel[_w8] at
 * inference_gpt2_opt.cu:302-303, 329), plus the dtype and the stream. */
int kvattn_append(void* kv_cache, float* kv_scale, const void* qkv,
                  int B, int NH, int hs, int maxT, const int* d_cur_len,
                  int kv_dtype, void* stream);

/* Short-context path: one workgroup per (b,h), scores staged in LDS.
 * Replaces attention_forward_kv_small (Inference_gpt2/attention_kvcache.cuh:453-459) and
 * attention_forward_kv_small_w8 (Inference_gpt2/attention_kvcache_w8.cuh:529-536). */
int kvattn_forward_small(void* out, const void* qkv, const void* kv_cache,
                         const float* kv_scale, int B, int NH, int hs, int maxT,
                         const int* d_cur_len, int lens_per_seq,
                         int kv_dtype, void* stream);

/* Long-context path with caller-owned partials of S segments per (b,h).  As in the
 * reference, B == 1 takes a single launch and B > 1 (or a capture) the split + merge pair
 * over the caller's partials.  The single launch is the designated merger (SPLIT_DESIGNATED
 * over the reference partition), not a cooperative launch: on this stack a cooperative
 * dispatch alone costs ~20 us of GPU time.  Its tagged partials live in the library's static
 * scratch array (the one kvattn_decode_static uses), so the call only enqueues: it allocates
 * nothing and never synchronises, as the reference's launches over caller-owned partials
 * (inference_gpt2_opt.cu:710-716).  S > 64, a grid the GPU cannot hold at once, or more than
 * about 9,200 slots (NH * S) take the split + merge pair instead.  Like kvattn_decode_static, calls
 * that overlap in time on one GPU (unordered streams, concurrent host threads) share the
 * array and may find each other's words: a merger never takes another call's word (each
 * carries its call's identity), but may wait for its bound and compute its producers'
 * segments itself (kvattn_scratch_status counts those).  Ordered calls, on one stream or
 * across streams, do not interfere.
 * Replaces attention_forward_kv_large (Inference_gpt2/attention_kvcache.cuh:464-487) and
 * attention_forward_kv_large_w8 (Inference_gpt2/attention_kvcache_w8.cuh:541-566). */
int kvattn_forward_large(void* out, const void* qkv, const void* kv_cache,
                         const float* kv_scale, int B, int NH, int hs, int maxT,
                         const int* d_cur_len, int lens_per_seq,
                         float* part_out, float* part_lse, float* part_max, int S,
                         int kv_dtype, void* stream);

/* Split phase alone: segment s of (b,h) covers [s*chunk, min((s+1)*chunk, total)) with
 * chunk = ceil(total/S); an empty segment writes (max=-FLT_MAX, lse=0, out=0).
 * Replaces the attention_kv_split_kernel[_w8] launches used under graph capture
 * (inference_gpt2_opt.cu:310-312,338-339; kernels at attention_kvcache.cuh:185-288 and
 * attention_kvcache_w8.cuh:260-363). */
int kvattn_split(float* part_out, float* part_lse, float* part_max,
                 const void* qkv, const void* kv_cache, const float* kv_scale,
                 int B, int NH, int hs, int maxT,
                 const int* d_cur_len, int lens_per_seq, int S,
                 int kv_dtype, void* stream);

/* Merge phase alone: out = sum_s e_s*part_out_s / sum_s e_s*part_lse_s with
 * e_s = exp(part_max_s - max_s part_max_s).  `out` is float when kv_dtype is F32, else
 * bfloat16.  Replaces the attention_kv_merge_kernel[_w8] launches
 * (inference_gpt2_opt.cu:313-314,340-341; kernels at attention_kvcache.cuh:298-318 and
 * attention_kvcache_w8.cuh:374-396). */
int kvattn_merge(void* out, const float* part_out, const float* part_lse,
                 const float* part_max, int B, int NH, int hs, int S,
                 int kv_dtype, void* stream);

/* Bytes of workspace kvattn_decode needs for (B, NH, hs, maxT, S).  S > 0 sizes for
 * exactly S segments per (b,h); S == 0 sizes for every automatic choice. */
size_t kvattn_workspace_bytes(int B, int NH, int hs, int maxT, int S);

/* Zero the workspace (merge counters, status words).  Call once after allocating a
 * workspace and before the first kvattn_decode on it; the kernels leave the counters at
 * zero after every call, and the designated merger's partial words carry the dispatch that
 * wrote them, so they never need clearing.  Enqueues one fill kernel (no hipMemsetAsync),
 * so it may also be captured. */
int kvattn_workspace_init(void* workspace, size_t workspace_bytes, void* stream);

/* The workspace's sticky status: waits for `stream`, then reads the number of merges that
 * stopped waiting since the workspace was initialised or last cleared.  A designated merger
 * (SPLIT_DESIGNATED, AUTO's latency-bound choice) that stops waiting for its producers
 * computes their segments itself, so its output is still the attention (only slower); a
 * cooperative merger that stops waiting at the grid barrier writes NaN for its (b,h).
 * *merge_timeouts (may be NULL) receives that number; clear != 0 resets it.
 * Returns KVATTN_ERR_MERGE_TIMEOUT when it is non-zero, else KVATTN_OK.  Partials left by
 * such a call are never taken for a later call's (each partial word carries the dispatch that
 * wrote it and that dispatch's hardware queue), so the workspace stays usable without
 * re-initialising.
 * No reference counterpart: the reference has no in-kernel wait that can give up, and
 * reports errors by exiting (common.h:123-130). */
int kvattn_workspace_status(void* workspace, size_t workspace_bytes, int clear, void* stream,
                            int* merge_timeouts);

/* kvattn_workspace_status for the library's static scratch array on the current device (the
 * workspace of kvattn_decode_static and of kvattn_forward_large's single launch): waits for
 * `stream`, then *merge_timeouts (may be NULL) receives the number of merges that stopped
 * waiting there since the array was first used or last cleared; clear != 0 resets it.
 * Returns KVATTN_ERR_MERGE_TIMEOUT when it is non-zero, else KVATTN_OK.
 * No reference counterpart (the reference has no in-kernel wait that can give up). */
int kvattn_scratch_status(int clear, void* stream, int* merge_timeouts);

/* Enqueue on `stream` one dispatch that writes the identity the tagged partial words of a
 * dispatch on that stream carry: out[0] its dispatch id (counted per hardware queue),
 * out[1] the address of its hardware queue, out[2] its 32-bit tag (the dispatch id plus a hash
 * of the queue address, top bit set).  out: 3 device words, 8-byte aligned.
 * No reference counterpart: a testing hook showing that calls on different streams, whose
 * dispatch ids coincide, never share a tag. */
int kvattn_call_identity(unsigned long long* out, void* stream);

/* Moves every designated producer of an XCD-local grid (8 or more (b,h) rows) `rot` XCDs
 * (mod 8) away from its merger, for launches (and captures) from this call on, process-wide;
 * 0 (the default) keeps each head's segments on one XCD.  Returns the previous setting.
 * Each designated merger publishes the XCD it runs on and each producer publishes its partial
 * with plain stores (which stay in its XCD's L2) only when that XCD is its own, else
 * write-through, so a producer placed elsewhere, by this setting or by a dispatcher that hands
 * workgroups to XCDs otherwise than the layout expects, costs the merger no wait: the output
 * and the merge-timeout count stay as they are.
 * No reference counterpart: a testing hook for the layout the designated merger relies on. */
int kvattn_set_xcd_layout_offset(int rot);

/* Bound on the polls of a designated merger waiting for its producers' partials (and of a
 * cooperative merger at the grid barrier), for launches (and captures) from this call on,
 * process-wide: polls > 0 sets it, polls == 0 makes every merger of a multi-segment (b,h)
 * stop waiting at once (a fault-injection setting, for testing the fallback and the
 * reporting above), polls < 0 restores the default (2^16 polls, tens of milliseconds).
 * Returns the previous bound.  No reference counterpart (testing and fault-injection hook). */
int kvattn_set_merge_poll_limit(int polls);

/* The launch plan kvattn_decode would use for these arguments, without launching:
 * *strategy_out = the resolved kvattn_strategy (AUTO resolved), *segments_out = segment
 * slots per (b,h) (1 for FUSED_SINGLE), *seg_rows_out = rows per segment (0 when the
 * reference partition ceil(total/S) is used, -1 when the kernels plan the rows from the
 * device length).  The plan is that of a call with one length for the batch
 * (lens_per_seq == 0).  A call with per-sequence lengths takes the same plan, except where
 * this one streams a BF16 or INT8 cache through the split + merge kernels: there AUTO keeps
 * its general plan (the last-block merge, or split + merge over segments of up to 512
 * rows).  No reference counterpart: it exposes the AUTO choice, which the reference makes
 * inline in its caller (inference_gpt2_opt.cu:247,304,331: fused_single below a length
 * threshold, split + merge above it). */
int kvattn_plan(int B, int NH, int hs, int maxT, int len_hint, int S, int strategy, int kv_dtype,
                int* strategy_out, int* segments_out, int* seg_rows_out);

/* One decode-attention call with an explicit strategy, the unified entry the per-layer
 * attention block of forward_kv_graph_ready (inference_gpt2_opt.cu:298-347) maps onto.
 *   strategy   kvattn_strategy; AUTO picks from len_hint (the host's view of cur_len,
 *              used for the choice only; -1 = unknown, treated as maxT-1).
 *   len_hint   -1 when the call must serve any length, as a graph captured once and
 *              replayed token after token: with S == 0 the kernels then plan the
 *              segmentation from the device length (one segment up to 256 positions,
 *              about four beyond, segments of at most 512 rows up to 64 of them, longer
 *              rows past 32768 positions), where the reference captures a small and a large
 *              graph and picks one per token (inference_gpt2_opt.cu:420-449,556).  AUTO
 *              with more than 16 heads (B*NH), or a longer maxT, takes fixed rows sized
 *              for maxT instead while its designated grid stays small (kvattn_plan
 *              reports them); segments past a call's length exit at once.
 *   S          segments per (b,h) for the split strategies: S > 0 uses the reference
 *              partition chunk = ceil(total/S); S < 0 uses -S rows per segment; S == 0
 *              lets the library pick the rows per segment (from len_hint, or on the
 *              device) and the per-sequence count from each length.
 *   workspace  device memory of kvattn_workspace_bytes(B, NH, hs, maxT, S) bytes,
 *              initialised once with kvattn_workspace_init; may be NULL for
 *              FUSED_SINGLE.  Calls sharing a workspace must be ordered: on one stream,
 *              or on several streams ordered by events (the designated merger's words
 *              carry the dispatch and its hardware queue, so a word another stream's call
 *              left is never taken for this call's).  Calls that overlap in time race.
 *   workspace_bytes  the buffer's actual size, the same for every call on the buffer.
 *              One buffer, sized for the largest plan, may serve calls of different
 *              plans (other B, NH or S): the last-block counters sit in a region whose
 *              size follows from workspace_bytes alone, the partials are laid out from
 *              the region's end and the designated merger's tagged words from the
 *              buffer's end, so no call finds its counters or tags where another left
 *              partials.
 */
int kvattn_decode(void* out, const void* qkv, const void* kv_cache, const float* kv_scale,
                  int B, int NH, int hs, int maxT,
                  const int* d_cur_len, int lens_per_seq, int len_hint,
                  void* workspace, size_t workspace_bytes,
                  int S, int strategy, int kv_dtype, void* stream);

/* kvattn_decode without a workspace argument: the partials, merge counters and tagged words
 * live in `scratch`, a static device array of 8 MiB that the library holds on each GPU it
 * runs on until the process ends, so the call allocates nothing (no hipMalloc, no hipFree;
 * a fill kernel clears the array's counters on its first call on a device).
 * No reference counterpart: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Limits: B*NH <= 16384, and the plan's partials and tagged words (kvattn_workspace_bytes
 * less its status words and counters) within 8 MiB - 64.25 KiB, else KVATTN_ERR_WORKSPACE;
 * strategies AUTO, FUSED_SINGLE, SPLIT_MERGE, SPLIT_LASTBLOCK, SPLIT_DESIGNATED (the
 * cooperative launch and the library's graph pair return KVATTN_ERR_STRATEGY: the runtime may
 * allocate for them).  Every call on one GPU shares that GPU's array (with
 * kvattn_forward_large's single launch), which keeps the last call's contents: calls that
 * overlap in time on one GPU (unordered streams, concurrent host threads) race; calls ordered
 * on one stream, or across streams by events, do not.  kvattn_scratch_status reads its merge
 * timeouts. */
int kvattn_decode_static(void* out, const void* qkv, const void* kv_cache, const float* kv_scale,
                         int B, int NH, int hs, int maxT,
                         const int* d_cur_len, int lens_per_seq, int len_hint,
                         int S, int strategy, int kv_dtype, void* stream);

/* kvattn_cache_write followed by kvattn_decode with the same arguments, in one launch
 * (two for SPLIT_MERGE): the current token's K and V rows are taken from qkv in registers
 * (8-bit: quantised exactly as kvattn_cache_write does), written into column cur_len, and
 * used in place of that cache column.  Cache contents and outputs equal those of the two
 * calls.  Replaces the append launch kv_cache_write_kernel[_w8] together with the attention
 * call after it (inference_gpt2_opt.cu:302-316, 329-345); the reference's ranked follow-up
 * removes the same launch by moving the append into the QKV GEMV epilogue instead. */
int kvattn_append_decode(void* out, const void* qkv, void* kv_cache, float* kv_scale,
                         int B, int NH, int hs, int maxT,
                         const int* d_cur_len, int lens_per_seq, int len_hint,
                         void* workspace, size_t workspace_bytes,
                         int S, int strategy, int kv_dtype, void* stream);

/* ---- Paged KV cache ------------------------------------------------------------------
 * No reference counterpart: the reference keeps one contiguous [2][B][NH][maxT][hs] cache
 * per layer and names paged KV management as its gap for multi-request serving
 * (README.md:62-63).  Here a layer's cache may instead be a pool of pages:
 *   pages        [num_pages][2][NH][page_rows][hs] elements (K block, then V block, of
 *                page_rows positions of one sequence for every head)
 *   page_scales  [num_pages][2][NH][page_rows] FP32 row scales (8-bit caches), else NULL
 *   block_table  [B][max_pages] int32: page id holding positions
 *                [i*page_rows, (i+1)*page_rows) of sequence b at block_table[b*max_pages+i]
 * page_rows is a multiple of 64; a sequence holds up to max_pages*page_rows positions
 * (the maxT of these calls).  Table entries outside [0, num_pages) are never dereferenced:
 * their positions are skipped (attention) or not written (append).  Row layout, element
 * types and 8-bit codes are those of the contiguous cache. */

/* kvattn_cache_write into a paged cache. */
int kvattn_paged_cache_write(void* pages, float* page_scales, const int* block_table,
                             int max_pages, int page_rows, int num_pages,
                             const void* qkv, int B, int NH, int hs,
                             const int* d_cur_len, int lens_per_seq, int kv_dtype, void* stream);

/* kvattn_decode (append == 0) or kvattn_append_decode (append != 0) on a paged cache.
 * Strategies: AUTO, SPLIT_MERGE, SPLIT_LASTBLOCK, SPLIT_DESIGNATED, SINGLE_LAUNCH_GRAPH (no
 * FUSED_SINGLE or cooperative launch: short contexts take a single segment of the split
 * kernel).  S == 0 plans the segments on the device, except where AUTO takes the designated
 * merger or one segment per (b,h) with fixed rows (128, 256 or 512: the choice kvattn_decode's
 * AUTO makes for a contiguous cache, hinted lengths of up to 256 positions excepted); S < 0
 * gives -S rows per segment, a multiple of 64 and at most 4096.  Workspace:
 * kvattn_workspace_bytes(B, NH, hs, max_pages*page_rows, S). */
int kvattn_paged_decode(void* out, const void* qkv, void* pages, float* page_scales,
                        const int* block_table, int max_pages, int page_rows, int num_pages,
                        int B, int NH, int hs,
                        const int* d_cur_len, int lens_per_seq, int len_hint,
                        void* workspace, size_t workspace_bytes,
                        int S, int strategy, int kv_dtype, int append, void* stream);

/* The decode step's fully connected layer, used after the attention for the output
 * projection: for b < B, m < M
 *   pre = w_scale[m] * sum_k W[m][k] * x[b][k] + bias[m]      (w_scale: 8-bit weights only)
 *   pre_gelu[b][m] = pre (if pre_gelu != NULL);  out[b][m] = gelu ? GELU_tanh(pre) : pre
 * with FP32 accumulation.  Types by w_dtype (a kvattn_dtype):
 *   F32        W, x, bias, out, pre_gelu float
 *   BF16       W, x, bias, out, pre_gelu bf16
 *   INT8, FP8  W one code per weight ([M][K] bytes) with one FP32 scale per row; x, bias,
 *              out, pre_gelu bf16
 * W is row-major [M][K]; x [B][K]; out [B][M].  Requires K % 16 == 0 (any length: rows
 * beyond 64 * 16 chunks of 16 bytes are walked in blocks, as the reference's tail loops walk
 * any K), 16-byte aligned W and x.  bias may be NULL.  From 8192 rows on (a vocabulary
 * projection), each wave takes 4 rows so that more weight bytes are in flight.
 * Replaces launch_GEMV6_fused (Inference_gpt2/GEMV.cuh:132-206) and launch_GEMV6_w8x2
 * (Inference_gpt2/GEMV_w8.cuh:64-184), which matmul_forward[_w8] calls for one decode token
 * (inference_gpt2_opt.cu:106-132); the attention output projection is at :349-355.  B > 1
 * reads the weights once for all B vectors when a row fits in one block (the reference
 * takes cuBLASLt there). */
int kvattn_gemv(void* out, void* pre_gelu, const void* W, const float* w_scale, const void* x,
                const void* bias, int B, int M, int K, int w_dtype, int gelu, void* stream);

/* kvattn_gemv with the output type given: out and pre_gelu are float (out_dtype
 * KVATTN_KV_F32) or bf16 (KVATTN_KV_BF16), whatever the weights; x and bias keep the
 * activation type of w_dtype.  Replaces the reference's instantiations with an output type
 * other than the activations', such as the vocabulary projection over the 8-bit embedding
 * table, launch_GEMV6_w8x2<float, floatX>(logits, NULL, w8_wte, lnf, w8_wte_s, NULL, Vp, C,
 * false, stream) (inference_gpt2_opt.cu:389-394). */
int kvattn_gemv_ex(void* out, void* pre_gelu, const void* W, const float* w_scale, const void* x,
                   const void* bias, int B, int M, int K, int w_dtype, int out_dtype, int gelu, void* stream);

/* The QKV projection with the KV append in its epilogue: kvattn_gemv with M = 3 * NH * hs
 * (no GELU) into qkv [B][3][NH][hs], whose K and V rows also go to column cur_len of
 * kv_cache [2][B][NH][maxT][hs], as kvattn_cache_write would write them, bit for bit.
 *   kv_dtype F32 / BF16: the cache holds the activation type (float for F32 weights, bf16
 *     otherwise); kv_scale and the workspace are not used.
 *   kv_dtype INT8 / FP8_E4M3 (bf16 activations): codes and one row scale per (b, K|V, h) in
 *     kv_scale [2][B][NH][maxT], from the bf16 values in qkv with the append's quantiser.
 *     The 64 channels of a row come from 16 workgroups, so they meet in the workspace:
 *     kvattn_gemv_qkv_append_workspace_bytes(B, NH) bytes, 256-byte aligned, zeroed once
 *     (kvattn_workspace_init); each word there carries the call that wrote it, so the
 *     workspace needs no clearing between calls.  Calls sharing a workspace must be ordered
 *     (one stream).
 * d_cur_len as in kvattn_decode (NULL: the library's device length).  hs must be 64.
 * Replaces the QKV GEMV followed by the append launch (inference_gpt2_opt.cu:290-303, 329;
 * the append kernels attention_kvcache.cuh:46-64, attention_kvcache_w8.cuh:115-155), one
 * launch fewer per layer. */
size_t kvattn_gemv_qkv_append_workspace_bytes(int B, int NH);
int kvattn_gemv_qkv_append(void* qkv, const void* W, const float* w_scale, const void* x,
                           const void* bias, int B, int NH, int hs, int K, void* kv_cache,
                           float* kv_scale, int maxT, const int* d_cur_len, int lens_per_seq,
                           int w_dtype, int kv_dtype, void* workspace, size_t workspace_bytes,
                           void* stream);

#ifdef __cplusplus
}
#endif
#endif /* KVATTN_H */
