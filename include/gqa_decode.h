/*
 * gqa_decode.h -- C ABI of the MI355X (gfx950) GQA paged-decode kernels.
 *
 * Single-token GQA decode attention over a paged bf16 KV cache, head dim 128:
 *
 *   out[b, h, :] = softmax_t( scale * <q[b, h, :], K_b[t, kv(h), :]> ) . V_b[t, kv(h), :]
 *   kv(h)        = h / (Hq / Hkv)                       (consecutive grouping)
 *   K_b[t]       = k_cache[block_table[b, t / block_size], t % block_size]
 *
 * Tensor layouts (all row-major, contiguous, device memory):
 *   q            [B, Hq, 128]                       bf16 (raw bits, uint16_t)
 *   k_cache      [num_blocks, block_size, Hkv, 128] bf16 (NHD)
 *   v_cache      [num_blocks, block_size, Hkv, 128] bf16 (NHD)
 *   block_table  [B, max_blocks]                    int32; entries at or beyond
 *                                                    ceil(seq_lens[b]/block_size)
 *                                                    are never read
 *   seq_lens     [B]                                int32, each >= 1
 *   out          [B, Hq, 128]                       bf16, round-to-nearest-even
 *
 * Every launcher is asynchronous on `stream`, allocates nothing, and returns
 * hipSuccess (0) or a hipError_t code: hipErrorInvalidValue (1) for arguments
 * it rejects before launching, otherwise the error hipGetLastError() reports
 * after the launch. seq_lens[b] == 0 is unsupported (the result is NaN, as in
 * the reference). All entry points are reentrant; results are bitwise
 * deterministic for identical inputs.
 *
 * Reference counterparts (paths relative to the reference checkout):
 *   gqa_decode_v0_launch   include/gqa_decode.h:6-10,  kernels/gqa_decode/v0_naive.cu:27-36
 *   gqa_decode_v1_launch   include/gqa_decode.h:12-16, kernels/gqa_decode/v1_vectorized.cu:73-82
 *   gqa_decode_v2_launch   include/gqa_decode.h:18-23, kernels/gqa_decode/v2_splitkv.cu:110-125
 * The names and argument order are the reference's; the differences are the
 * C linkage, HIP stream type, bf16 passed as raw uint16_t bits, and the
 * int error code in place of void.
 */
#ifndef GQA_DECODE_H_
#define GQA_DECODE_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Entry points are the only symbols the library exports. */
#define GQA_DECODE_API __attribute__((visibility("default")))

/* Head dimension the kernels are built for. */
#define GQA_DECODE_HEAD_DIM 128
/* Largest num_splits gqa_decode_v2_launch accepts (python/gqa_decode_ext.cpp:102-103). */
#define GQA_DECODE_MAX_SPLITS 512

/* v0: correctness-first kernel, one wave64 per (b, q-head), token-serial online
 * softmax. Replaces gqa_decode_v0_launch (include/gqa_decode.h:6-10). */
GQA_DECODE_API int gqa_decode_v0_launch(const uint16_t* q, const uint16_t* k_cache,
                         const uint16_t* v_cache, const int* block_table,
                         const int* seq_lens, uint16_t* out, int B, int Hq,
                         int Hkv, int block_size, int max_blocks, float scale,
                         hipStream_t stream);

/* v1: single-pass scan, one workgroup per (b, kv-head) holding the whole
 * q-head group, 16-byte row loads, fp32 online-softmax state. Groups of 5-16
 * q-heads over 4 or 8 kv-heads run the matrix-core scan, one workgroup per
 * request with a wave per kv-head, when the batch alone fills the device
 * (B * Hkv * 4 >= 24 * CUs). Groups of up to 4 q-heads run it too when the
 * grid leaves CUs idle (B * Hkv < CUs) and max_blocks * block_size is at most
 * 1024 tokens; such grids also give each workgroup up to 12 or 16 waves (8
 * on the matrix-core scan). Replaces gqa_decode_v1_launch
 * (include/gqa_decode.h:12-16). */
GQA_DECODE_API int gqa_decode_v1_launch(const uint16_t* q, const uint16_t* k_cache,
                         const uint16_t* v_cache, const int* block_table,
                         const int* seq_lens, uint16_t* out, int B, int Hq,
                         int Hkv, int block_size, int max_blocks, float scale,
                         hipStream_t stream);

/* v2: split-KV. A partial kernel writes one unnormalised fp32 (m, l, acc) state
 * per (b, q-head, split) to the caller's workspace, then a log-sum-exp merge
 * kernel writes `out`. Which scan runs depends on the shape, num_splits and the
 * device's CU count (the layout rule of gqa_decode_v1_launch with
 * B * num_splits in place of B), so results are bitwise reproducible for the
 * same inputs, split count and device. For groups of up to 4 q-heads, once
 * num_splits reaches 4 * max(1, CUs / (B * Hkv)) -- the waves the launch gives
 * each (request, kv-head) pair -- every split is scanned by one wave, each
 * wave walking a run of consecutive splits; with one workgroup per pair
 * (B * Hkv >= CUs) and at most 19 splits per wave (37 for 2-head groups, 74
 * for 1-head groups, 25 for 3-head groups) that workgroup also merges its
 * splits, and no merge kernel runs. out is bitwise equal to
 * gqa_decode_v2_partial_launch followed by gqa_decode_v2_merge_launch in every
 * case, and the workspace holds the same states. Workspace layout (the reference's, v2_splitkv.cu:10-12):
 *   ws_acc [B, Hq, num_splits, 128] fp32, ws_m / ws_l [B, Hq, num_splits] fp32
 * ws_m holds the segment's max of scale*<q,k> (natural-log units), ws_l the sum
 * of exp(score - ws_m), ws_acc the exp-weighted sum of V rows.
 * Split rule: split i of request b covers tokens [i*chunk, min(S_b, (i+1)*chunk))
 * with chunk = ceil(S_b / num_splits) rounded UP to a multiple of 32 tokens.
 * The reference uses chunk = ceil(S_b / num_splits) unrounded
 * (v2_splitkv.cu:30-32): the rounding keeps each 16-token tile inside one
 * cache block, so for short sequences the trailing splits can be empty
 * (S = 100, num_splits = 8: chunk 32, splits 0-3 live, 4-7 empty; the
 * reference's chunk would be 13 with all 8 live). A caller that produces or
 * consumes per-split states itself must use this rule. An empty segment
 * stores (-inf, 0, 0). num_splits must be in [1, GQA_DECODE_MAX_SPLITS];
 * num_splits == 1 gives output bitwise equal to gqa_decode_v1_launch.
 * Replaces gqa_decode_v2_launch (include/gqa_decode.h:18-23). */
GQA_DECODE_API int gqa_decode_v2_launch(const uint16_t* q, const uint16_t* k_cache,
                         const uint16_t* v_cache, const int* block_table,
                         const int* seq_lens, uint16_t* out, int B, int Hq,
                         int Hkv, int block_size, int max_blocks, float scale,
                         int num_splits, float* ws_acc, float* ws_m,
                         float* ws_l, hipStream_t stream);

/* The two halves of gqa_decode_v2_launch, for callers that produce or combine
 * split states themselves (e.g. a context-parallel decode that all-gathers
 * partial states across devices and then merges them). Same arguments and
 * workspace contract as gqa_decode_v2_launch; _partial writes only the
 * workspace, _merge reads only the workspace (any num_splits states per
 * (b, q-head), in whatever token split the caller chose, fold correctly; the
 * partial kernel's own split is the 32-token-rounded rule above). Reference counterparts: the
 * partial and merge launches inside gqa_decode_v2_launch
 * (kernels/gqa_decode/v2_splitkv.cu:115-124). */
GQA_DECODE_API int gqa_decode_v2_partial_launch(const uint16_t* q, const uint16_t* k_cache,
                                 const uint16_t* v_cache, const int* block_table,
                                 const int* seq_lens, int B, int Hq, int Hkv,
                                 int block_size, int max_blocks, float scale,
                                 int num_splits, float* ws_acc, float* ws_m,
                                 float* ws_l, hipStream_t stream);

GQA_DECODE_API int gqa_decode_v2_merge_launch(const float* ws_acc, const float* ws_m,
                               const float* ws_l, uint16_t* out, int B, int Hq,
                               int num_splits, hipStream_t stream);

/* Bytes of workspace gqa_decode_v2_launch needs for (B, Hq, num_splits), all
 * three arrays together: B*Hq*num_splits*(128 + 2)*4. Returns 0 for
 * non-positive arguments. No reference counterpart (the reference sizes the
 * workspace inline at python/gqa_decode_ext.cpp:106-109). */
GQA_DECODE_API size_t gqa_decode_v2_workspace_bytes(int B, int Hq, int num_splits);

/* Single-launch split-KV: gqa_decode_v2_launch's result in one kernel launch.
 * The partial kernel runs with the same split rule and layout; the last
 * workgroup of each merge group (a request's q-heads on one kv-head) to
 * finish its split folds the group's states in split order with the merge
 * kernel's arithmetic, so out is bitwise equal to gqa_decode_v2_launch's with
 * the same num_splits. workspace (16-byte aligned, workspace_bytes at least
 * gqa_decode_v2_fused_workspace_bytes) starts with B*Hq 32-bit arrival
 * counters and ends with the v2 workspace (ws_acc, ws_m, ws_l back to back,
 * as gqa_decode_v2_launch takes them), placed at the last 256-byte boundary
 * that leaves room for it. The counters must be zero before the first launch
 * (gqa_decode_v2_fused_reset for the largest B*Hq the workspace will serve);
 * every launch leaves them zero, so one workspace serves any smaller batch
 * afterwards. Launches that share a workspace must not overlap (stream order
 * suffices). No workgroup waits on another. num_splits == 1 runs the
 * single-pass kernel; where gqa_decode_v2_launch merges inside its one
 * workgroup per pair (see above), this launch does the same and leaves the
 * counters untouched. Cost elsewhere: each arriving workgroup writes back its
 * L2 lines (the release of the arrival count), about 300 ns of its XCD's L2
 * time, so the launch pays off with a few hundred arriving workgroups (one
 * 8192-token request at 32 splits: 16.6 us against 19.9 us for two launches)
 * and loses past a thousand (2048 arriving workgroups, 32 requests of 8192
 * tokens at 8 splits with 4 waves per split: 255 us against 173 us); prefer
 * gqa_decode_v2_launch when more than about a thousand workgroups would
 * arrive.
 * No reference counterpart: the reference's v2 is a
 * partial and a merge launch (kernels/gqa_decode/v2_splitkv.cu:110-125) and
 * lists the fused merge as a follow-up (README.md:386-387, 410-412). */
GQA_DECODE_API int gqa_decode_v2_fused_launch(const uint16_t* q, const uint16_t* k_cache,
                                              const uint16_t* v_cache, const int* block_table,
                                              const int* seq_lens, uint16_t* out, int B, int Hq,
                                              int Hkv, int block_size, int max_blocks,
                                              float scale, int num_splits, void* workspace,
                                              size_t workspace_bytes, hipStream_t stream);

/* Bytes of workspace gqa_decode_v2_fused_launch needs: 4*B*Hq rounded up to
 * a multiple of 256, plus gqa_decode_v2_workspace_bytes(B, Hq, num_splits); 0
 * for non-positive arguments. */
GQA_DECODE_API size_t gqa_decode_v2_fused_workspace_bytes(int B, int Hq, int num_splits);

/* Zero the arrival counters of a fused-launch workspace for (B, Hq) -- the
 * first 4*B*Hq bytes, rounded up to 256 -- with a fill kernel on stream (no
 * memset node, so it can be captured in a graph). Call once after allocating
 * the workspace. num_splits only sizes the workspace check. */
GQA_DECODE_API int gqa_decode_v2_fused_reset(void* workspace, size_t workspace_bytes, int B,
                                             int Hq, int num_splits, hipStream_t stream);

/* Split count that fills the device. Groups of 5-16 q-heads over 4 or 8
 * kv-heads: one workgroup of Hkv waves per CU (B * Hkv * splits = 8 * CUs,
 * rounded down), no split longer than 4096 tokens nor shorter than 1024, at
 * most 32 splits -- when that grid fills at least 3/4 of the CUs. Otherwise:
 * as many (b, kv-head, split) waves as fit one round of one wave per SIMD (two
 * for the matrix-core scan on sequences of 8192+ tokens), no split longer than
 * 8192 tokens, each wave keeping at least two 16-token tiles, and at most 32
 * splits. max_blocks*block_size is taken as the longest sequence. num_cus <= 0 means
 * "query the current device". Returns a value in [1, 32], or 0 for invalid
 * arguments. No reference counterpart: the reference defaults to 8
 * (python/gqa_decode_ext.cpp:133) and picks the best value by sweep
 * (bench/run_matrix.py:84-94). Pure host code. */
GQA_DECODE_API int gqa_decode_pick_num_splits(int B, int Hq, int Hkv, int block_size,
                               int max_blocks, int num_cus);

/* Largest GQA group (Hq / Hkv) the token-balanced launcher serves: up to 16
 * q-heads with 4 or 8 kv-heads (matrix-core scan), up to 4 with other kv-head
 * counts (VALU scan). */
#define GQA_DECODE_BALANCED_MAX_GROUP 16
/* Largest batch the token-balanced launcher serves. */
#define GQA_DECODE_BALANCED_MAX_BATCH 20479

/* Token-balanced split-KV: a persistent grid of num_workgroups workgroups
 * (<= 0: one per CU of the current device), each taking an equal share of the
 * batch's 16-token tiles, whatever the lengths -- in request order on the
 * matrix-core scan (one wave per kv-head) for 4 or 8 kv-heads, in
 * (request, kv-head) order on the VALU scan for other kv-head counts (groups
 * of up to 4 q-heads); segments cut at a share boundary are merged by a second
 * kernel in share order, so results are bitwise reproducible for a given
 * num_workgroups (and agree with v1/v2 within rounding, not bitwise). The host
 * never reads seq_lens. Lengths are clamped to max_blocks * block_size; a
 * request of length 0 gets NaN. Requires Hq / Hkv <=
 * GQA_DECODE_BALANCED_MAX_GROUP (with Hkv 4 or 8 for groups of 5+) and
 * B <= GQA_DECODE_BALANCED_MAX_BATCH (else hipErrorInvalidValue), and a
 * workspace of at least gqa_decode_balanced_workspace_bytes() bytes, 16-byte
 * aligned, whose contents need no initialisation. No reference counterpart:
 * the reference's split count is per request (kernels/gqa_decode/
 * v2_splitkv.cu:30-32); this is its split-KV with splits sized by tokens. */
GQA_DECODE_API int gqa_decode_balanced_launch(const uint16_t* q, const uint16_t* k_cache,
                               const uint16_t* v_cache, const int* block_table,
                               const int* seq_lens, uint16_t* out, int B, int Hq,
                               int Hkv, int block_size, int max_blocks, float scale,
                               int num_workgroups, float* workspace,
                               size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes gqa_decode_balanced_launch needs: two partial states and a
 * small share record per workgroup. 0 for invalid arguments or an unsupported
 * group size. */
GQA_DECODE_API size_t gqa_decode_balanced_workspace_bytes(int B, int Hq, int Hkv,
                                                          int num_workgroups);

/* The two launches of gqa_decode_balanced_launch, same arguments: _partial
 * scans every share (writing `out` for whole segments, the workspace for cut
 * ones), _merge combines the cut segments into `out`. Issued in that order on
 * one stream they are gqa_decode_balanced_launch; separately they let a
 * caller time or profile the scan alone. */
GQA_DECODE_API int gqa_decode_balanced_partial_launch(
    const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, const int* block_table,
    const int* seq_lens, uint16_t* out, int B, int Hq, int Hkv, int block_size, int max_blocks,
    float scale, int num_workgroups, float* workspace, size_t workspace_bytes,
    hipStream_t stream);

GQA_DECODE_API int gqa_decode_balanced_merge_launch(
    const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, const int* block_table,
    const int* seq_lens, uint16_t* out, int B, int Hq, int Hkv, int block_size, int max_blocks,
    float scale, int num_workgroups, float* workspace, size_t workspace_bytes,
    hipStream_t stream);

/* Size of the device array gqa_decode_balanced_launch_noalloc uses as its
 * workspace: 32 MiB per device (two fp32 states of all q-heads per workgroup:
 * up to 64 q-heads at 256 workgroups). */
#define GQA_DECODE_NOALLOC_SCRATCH_BYTES (32u << 20)

/* gqa_decode_balanced_launch without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No reference counterpart: the
 * reference's launchers take caller-owned buffers and have no such variant.
 * Its workspace is a file-scope device array of
 * GQA_DECODE_NOALLOC_SCRATCH_BYTES in the library, one copy per device
 * (resolved for the stream's device on the first call there, and held until
 * the process ends); the call allocates nothing. num_workgroups <= 0 means the
 * CU count of the stream's device (the device whose array is used). Same
 * arguments, kernels and bits as gqa_decode_balanced_launch with the same
 * num_workgroups. The first call on a device must not be made while the
 * stream is being captured into a graph (it returns
 * hipErrorStreamCaptureUnsupported, launching nothing): make one eager call
 * per device first; later calls can be captured. Returns
 * hipErrorOutOfMemory, launching nothing, when
 * gqa_decode_balanced_workspace_bytes(B, Hq, Hkv, num_workgroups) exceeds
 * GQA_DECODE_NOALLOC_SCRATCH_BYTES; otherwise as gqa_decode_balanced_launch.
 * Every call on a device shares that device's array: calls that overlap on
 * one device (different streams without ordering, or threads) race and give
 * wrong results; calls in one stream's order do not. The array needs no
 * clearing: every byte a launch reads, it wrote. */
GQA_DECODE_API int gqa_decode_balanced_launch_noalloc(
    const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, const int* block_table,
    const int* seq_lens, uint16_t* out, int B, int Hq, int Hkv, int block_size, int max_blocks,
    float scale, int num_workgroups, hipStream_t stream);

/* 1 if gqa_decode_balanced_launch is expected to beat the split-KV launch with
 * gqa_decode_pick_num_splits' count for this shape on num_cus CUs (<= 0: the
 * current device), else 0 (also for shapes the balanced launcher does not
 * serve). The rule, from measurements on MI355X, with KV bytes counted at the
 * longest sequence (max_blocks * block_size) for every request. Groups of at
 * most 4 q-heads: a longest sequence of at least 6144 tokens, at least 32 MiB
 * of KV, at most 16 (request, kv-head) segments per CU, and not a split grid
 * of exactly one wave per SIMD with at most 8 splits (which uniform lengths
 * make perfectly even), and at least 8 requests when there are 4 or 8
 * kv-heads (the balanced launch then cuts whole requests into pieces). Groups
 * of 5-16 q-heads over 4 or 8 kv-heads: at least 8 requests and 512 MiB of
 * KV. This is the choice the torch op makes for
 * num_splits=0. Pure host code. No reference counterpart. */
GQA_DECODE_API int gqa_decode_prefer_balanced(int B, int Hq, int Hkv, int block_size,
                                              int max_blocks, int num_cus);

#ifdef __cplusplus
}
#endif

#endif /* GQA_DECODE_H_ */
