/*
 * mla_decode.h -- C ABI of the MI355X (gfx950) MLA absorbed-path paged decode.
 *
 * The reference's roadmap item K2 (README.md:405-408 of the reference): decode
 * attention of multi-head latent attention in its absorbed form, where every
 * query head attends over one shared latent cache whose rows hold the
 * compressed KV (512 dims) followed by the rotary key part (64 dims):
 *
 *   out[b, i, h, :] = softmax_t( scale * <q[b, i, h, :], C_b[t, :]> ) . C_b[t, :512]
 *   lse[b, h, i]    = log sum_t exp( scale * <q[b, i, h, :], C_b[t, :]> )   (natural log)
 *   C_b[t]          = kv_cache[block_table[b, t / block_size], t % block_size, 0, :]
 *
 * for t < seq_lens[b]; with causal != 0, query token i of s_q attends only to
 * t < seq_lens[b] - (s_q - 1 - i). The reference has no implementation (its
 * kernels/mla_decode/ is empty); the semantics and tensor layouts are those of
 * its pinned baseline, FlashMLA at 15f13e5 (docs/g0/flashmla_sha.txt):
 * flash_mla_with_kvcache(q, k_cache, block_table, cache_seqlens, head_dim_v,
 * tile_scheduler_metadata, num_splits, softmax_scale, causal) -> (out, lse).
 *
 * Layouts (row-major, contiguous, device memory; bf16 as raw uint16_t bits):
 *   q            [B, s_q, h_q, 576]               bf16
 *   kv_cache     [num_blocks, block_size, 1, 576] bf16 (one latent "head")
 *   block_table  [B, max_blocks]                  int32
 *   seq_lens     [B]                              int32, >= 0
 *   out          [B, s_q, h_q, 512]               bf16, round-to-nearest-even
 *   lse          [B, h_q, s_q]                    fp32
 * A query row with no key to attend (seq_lens[b] == 0, or causal rows past
 * the length) gets out = 0 and lse = -inf.
 *
 * Launchers are asynchronous on `stream`, allocate nothing and return 0 or a
 * hipError_t code (hipErrorInvalidValue for arguments rejected before any
 * launch). Results are bitwise deterministic for identical inputs and split
 * count. No reference counterpart beyond the roadmap entry cited above.
 */
#ifndef MLA_DECODE_H_
#define MLA_DECODE_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef GQA_DECODE_API
#define GQA_DECODE_API __attribute__((visibility("default")))
#endif

/* Head dimensions the kernels are built for: query/key (latent + rotary) and
 * value (latent). */
#define MLA_DECODE_HEAD_DIM 576
#define MLA_DECODE_HEAD_DIM_V 512
/* Largest num_splits accepted. */
#define MLA_DECODE_MAX_SPLITS 128

/* Split-KV MLA decode. A partial kernel writes one unnormalised fp32 state per
 * (request, query row, split) to the workspace; a merge kernel folds the
 * splits in order into out and lse. num_splits == 1 runs the partial kernel
 * alone, writing out and lse directly. Splits cut each request at multiples of
 * 32 tokens (chunk = ceil(S / num_splits) rounded up to 32). workspace:
 * mla_decode_workspace_bytes(B, s_q, h_q, num_splits) bytes, 16-byte aligned,
 * uninitialised is fine (none needed for num_splits == 1). */
GQA_DECODE_API int mla_decode_launch(const uint16_t* q, const uint16_t* kv_cache,
                                     const int* block_table, const int* seq_lens,
                                     uint16_t* out, float* lse, int B, int s_q, int h_q,
                                     int block_size, int max_blocks, float scale, int causal,
                                     int num_splits, void* workspace, size_t workspace_bytes,
                                     hipStream_t stream);

/* The two launches of mla_decode_launch, for a caller that schedules them
 * itself (or times them apart): the split kernel alone (same arguments; with
 * num_splits == 1 it writes out and lse, else the workspace states), then the
 * combine kernel, which folds the num_splits states of every (request, query
 * row) from the workspace into out and lse (num_splits >= 2; same workspace
 * and sizes as the split launch). Like FlashMLA's split and combine kernels,
 * which its single call runs back to back. */
GQA_DECODE_API int mla_decode_splitkv_launch(const uint16_t* q, const uint16_t* kv_cache,
                                             const int* block_table, const int* seq_lens,
                                             uint16_t* out, float* lse, int B, int s_q, int h_q,
                                             int block_size, int max_blocks, float scale,
                                             int causal, int num_splits, void* workspace,
                                             size_t workspace_bytes, hipStream_t stream);
GQA_DECODE_API int mla_decode_combine_launch(void* workspace, size_t workspace_bytes,
                                             uint16_t* out, float* lse, int B, int s_q, int h_q,
                                             int num_splits, hipStream_t stream);

/* Token-balanced MLA decode: the same results as mla_decode_launch (to
 * rounding), with the batch's work cut into equal shares whatever the lengths,
 * as FlashMLA's tile scheduler does. The work is every request's 32-token
 * tiles in request order (T = sum_b ceil(S_b / 32)); each of the ceil(s_q h_q
 * / 128) row groups gets n = num_workgroups / row groups shares
 * (num_workgroups <= 0: the device's CU count), share w taking tiles
 * [w T / n, (w + 1) T / n). Two launches on `stream`: the split kernel, each
 * of whose workgroups plans the launch from seq_lens on the device (tile
 * prefix sums, its share and first request: no host synchronisation,
 * graph-capturable; requests that fall inside one share are written to out
 * and lse directly, the pieces of the others to workspace states), and a
 * merge of the cut requests in share order (bitwise reproducible for a given
 * num_workgroups).
 * workspace: mla_decode_balanced_workspace_bytes(B, s_q, h_q, num_workgroups)
 * bytes, 16-byte aligned, uninitialised is fine. */
GQA_DECODE_API int mla_decode_balanced_launch(const uint16_t* q, const uint16_t* kv_cache,
                                              const int* block_table, const int* seq_lens,
                                              uint16_t* out, float* lse, int B, int s_q, int h_q,
                                              int block_size, int max_blocks, float scale,
                                              int causal, int num_workgroups, void* workspace,
                                              size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes for mla_decode_balanced_launch (0 for invalid arguments):
 * two states of s_q * h_q rows x (512 + 2) floats per share, then the tile
 * prefix sums (B + 2 uint64). */
GQA_DECODE_API size_t mla_decode_balanced_workspace_bytes(int B, int s_q, int h_q,
                                                          int num_workgroups);

/* Workspace bytes for mla_decode_launch: B * s_q * h_q * num_splits * (512 + 2)
 * * 4 for num_splits > 1, 0 for num_splits == 1 or invalid arguments. */
GQA_DECODE_API size_t mla_decode_workspace_bytes(int B, int s_q, int h_q, int num_splits);

/* Split count that gives every CU a workgroup of query rows: the smallest
 * count whose (row group, request, split) grid covers num_cus workgroups,
 * with splits of at least 256 tokens of the longest sequence
 * (max_blocks * block_size) and at most MLA_DECODE_MAX_SPLITS. num_cus <= 0:
 * the current device. Pure host code. */
GQA_DECODE_API int mla_decode_pick_num_splits(int B, int s_q, int h_q, int block_size,
                                              int max_blocks, int num_cus);

#ifdef __cplusplus
}
#endif

#endif /* MLA_DECODE_H_ */
