/*
 * minivllm_hip.h -- C ABI of libminivllm_hip.so, the MI355X (gfx950) paged-KV
 * decode hot path of the minivllm runtime.
 *
 * Plain C: raw device pointers, element strides, sizes and enums. No torch
 * types. Every compute entry point is asynchronous on the given HIP stream
 * (NULL = the legacy default stream) and returns an int status:
 *
 *   MGI_OK (0)           launched (or nothing to do)
 *   MGI_EINVAL (-1)      an argument violates the contract (shape, stride,
 *                        alignment, range, null pointer)
 *   MGI_EUNSUPPORTED(-2) a valid request this library does not implement
 *   MGI_ELAUNCH (-3)     the HIP runtime refused the launch
 *   MGI_EWORKSPACE (-4)  workspace missing or smaller than required
 *
 * On a non-zero status, mgi_last_error() returns a thread-local message.
 * No entry point synchronises the stream or reads device data on the host:
 * device-data invariants (context lengths >= 1, valid block-table entries for
 * every block a context touches) are the caller's, exactly as for the
 * reference backends. The kernels never read or write outside the buffers
 * described by the sizes given: out-of-range slots, block ids and context
 * lengths are skipped or clamped on the device.
 *
 * Layouts (element strides, row-major by default):
 *   KV pool      [L, N, S, H, D]   (KVBlockPool.k / .v)
 *   q, out       [B, H, D]         (any strides)
 *   k_new, v_new [T, H, D]         (any strides; T rows written)
 *   block_tables [B, M]            (int32 or int64; -1 padding in the tail)
 *   context_lens [B]               (int32 or int64; includes the new token)
 *   slot_mapping [T]               (int32 or int64; slot = block*S + offset;
 *                                   a negative slot means "skip this row")
 */
#ifndef MINIVLLM_HIP_H
#define MINIVLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum mgi_status {
  MGI_OK = 0,
  MGI_EINVAL = -1,
  MGI_EUNSUPPORTED = -2,
  MGI_ELAUNCH = -3,
  MGI_EWORKSPACE = -4
};

/* Element types of q / out / KV pool / new K,V. */
enum mgi_dtype { MGI_F32 = 0, MGI_BF16 = 1, MGI_F16 = 2 };

/* Element types of block tables, context lengths and slot mappings. */
enum mgi_itype { MGI_I32 = 0, MGI_I64 = 1 };

/* Thread-local description of the last failing call ("" if none). */
const char* mgi_last_error(void);

/* ABI version of this library (major*100 + minor). 1.01 added
 * mgi_paged_decode_balanced_waves and the even split of split_tokens = 0;
 * 1.02 the prefill key split (mgi_paged_prefill's workspace arguments and
 * mgi_paged_prefill_workspace_bytes); 1.03 mgi_paged_decode_noalloc; 1.04
 * mgi_paged_decode_append. */
int mgi_abi_version(void);

/*
 * KV append / scatter.
 * Replaces the inline decode KV write of
 * KVCacheCausalSelfAttention.forward_decode_batch
 * (minivllm/attention.py:370-392: physical_blocks = slots // S,
 * block_offsets = slots % S, pool.k[layer, blk, off] = k, same for v) and the
 * per-token prefill write loop that calls KVBlockPool.write_layer
 * (minivllm/attention.py:190-208, minivllm/kv_block_pool.py:91-109).
 *
 * For every row t < T with s = slot_mapping[t] and 0 <= s < N*S:
 *   k_pool[layer_idx, s / S, s % S, :, :] = k_new[t, :, :]
 *   v_pool[layer_idx, s / S, s % S, :, :] = v_new[t, :, :]
 * Rows with s < 0 (padding) or s >= N*S are skipped; nothing else in the pool
 * is touched. With new_dtype == pool_dtype the copy is bit-exact; otherwise
 * the value is converted with round-to-nearest-even (f32 -> bf16/f16) or
 * exactly (bf16/f16 -> f32). Other conversions return MGI_EUNSUPPORTED.
 * If two rows name the same slot, which one lands is unspecified (as for
 * torch index_put_ without accumulate).
 */
int mgi_kv_append(void* k_pool, void* v_pool,
                  const int64_t* k_pool_strides, /* [5] */
                  const int64_t* v_pool_strides, /* [5] */
                  int pool_dtype,
                  const void* k_new, const void* v_new,
                  const int64_t* k_new_strides, /* [3] */
                  const int64_t* v_new_strides, /* [3] */
                  int new_dtype,
                  const void* slot_mapping, int64_t slot_stride, int slot_itype,
                  int64_t T, int64_t H, int64_t D,
                  int64_t S, int64_t N, int64_t L, int64_t layer_idx,
                  void* stream);

/*
 * Paged decode attention (one query token per sequence).
 * Replaces paged_attention_batch_online_v1
 * (minivllm/paged_attention_batch.py:121-278) and
 * paged_attention_batch_triton_v0 / _paged_decode_f32
 * (minivllm/triton_paged_decode.py:29-155).
 *
 * For b < B, h < H, with c = context_lens[b] (clamped to [0, M*S]):
 *   out[b,h,:] = sum_t softmax_t(scale * q[b,h,:] . K[t,h,:]) * V[t,h,:]
 * over the c logical tokens t, where token t lives in physical block
 * block_tables[b, t / S] at offset t % S of layer layer_idx. Only those
 * tokens are read: table entries past ceil(c/S) are never loaded and slots
 * past c are never dereferenced. A table entry outside [0, N) inside the
 * context is treated as a fully masked block. c == 0 gives out = 0 (the
 * online_v1 result for a row with no active block).
 * q, out and the pool share one dtype; arithmetic is fp32.
 *
 * split_tokens: 0 lets the library split the work. When a table is wider
 * than one partition and B <= 4096 it splits evenly: the blocks of all
 * sequences, in sequence order, are cut into equal segments, one per
 * wavefront of a fixed count (mgi_paged_decode_balanced_waves), whatever the
 * spread of context lengths; each wavefront streams most of its segment and
 * the rest of every segment goes, in small runs, to whichever wavefronts
 * finish first. Otherwise, and for split_tokens > 0 (rounded to a multiple
 * of S), each context is cut into partitions of split_tokens tokens. Either
 * way, a sequence whose work is split writes (max, sum, unnormalised output)
 * partials that a second pass merges. The output does not depend on which
 * wavefront streams which run: calls with the same inputs give the same
 * bits.
 * workspace must hold mgi_paged_decode_workspace_bytes(...) bytes for the
 * same (B, H, D, S, M, split_tokens); it may be NULL when that is 0. Its
 * contents need no initialisation and are not meaningful after the call.
 * Calls that overlap in time (other streams) need separate workspaces.
 */
int mgi_paged_decode(void* out, const int64_t* out_strides, /* [3] */
                     const void* q, const int64_t* q_strides, /* [3] */
                     const void* k_pool, const void* v_pool,
                     const int64_t* k_pool_strides, /* [5] */
                     const int64_t* v_pool_strides, /* [5] */
                     int dtype,
                     const void* block_tables, const int64_t* bt_strides, /* [2] */
                     int bt_itype,
                     const void* context_lens, int64_t cl_stride, int cl_itype,
                     int64_t B, int64_t H, int64_t D, int64_t S, int64_t N,
                     int64_t M, int64_t L, int64_t layer_idx,
                     float scale, int64_t split_tokens,
                     void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * One decode step's KV append and attention in one call: mgi_kv_append of the
 * B rows k_new[b], v_new[b] ([B, H, D]) into slots slot_mapping[b] ([B]),
 * then mgi_paged_decode, on the same stream. Replaces the slot write and the
 * backend call of KVCacheCausalSelfAttention.forward_decode_batch
 * (minivllm/attention.py:370-416), which the reference issues one after the
 * other.
 *
 * Contract beyond the two calls': a slot that some sequence's context reads
 * must be the slot of its own row's last context position (block_tables[b,
 * (c-1)/S]*S + (c-1)%S, c = context_lens[b] clamped as in mgi_paged_decode),
 * as in decode, where row b holds sequence b's newest token. Negative slots,
 * slots outside the pool and slots no context reads are free. Under it the
 * pool and out are bit-identical to those of the two calls.
 *
 * On the fast path, with new_dtype == dtype, a unit head-dim stride and
 * 16-byte aligned rows, the append runs inside the attention launch: the
 * wavefront that streams a sequence's last block writes that row's slot
 * first (one launch fewer per step). Otherwise the append kernel runs first
 * (conversions as mgi_kv_append). Workspace as mgi_paged_decode for the same
 * sizes. Added in ABI 1.04.
 */
int mgi_paged_decode_append(void* out, const int64_t* out_strides, /* [3] */
                            const void* q, const int64_t* q_strides, /* [3] */
                            void* k_pool, void* v_pool,
                            const int64_t* k_pool_strides, /* [5] */
                            const int64_t* v_pool_strides, /* [5] */
                            int dtype,
                            const void* k_new, const void* v_new,
                            const int64_t* k_new_strides, /* [3] */
                            const int64_t* v_new_strides, /* [3] */
                            int new_dtype,
                            const void* slot_mapping, int64_t slot_stride, int slot_itype,
                            const void* block_tables, const int64_t* bt_strides, /* [2] */
                            int bt_itype,
                            const void* context_lens, int64_t cl_stride, int cl_itype,
                            int64_t B, int64_t H, int64_t D, int64_t S, int64_t N,
                            int64_t M, int64_t L, int64_t layer_idx,
                            float scale, int64_t split_tokens,
                            void* workspace, size_t workspace_bytes,
                            void* stream);

/*
 * mgi_paged_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference.
 * Same arguments (minus workspace and workspace_bytes), checks, kernels and
 * results as mgi_paged_decode; the split workspace is a 32 MiB array the
 * library holds on every device it runs on, for the life of the process
 * (resolved on the first call per device; nothing is allocated, here or
 * later). A call whose split needs more than that
 * (mgi_paged_decode_workspace_bytes > 32 MiB; the automatic split needs
 * about 13 MiB at head_dim 128 whatever B and the context lengths, explicit
 * small partitions over many long contexts can need more) returns
 * MGI_EUNSUPPORTED without launching. All calls on one device share the
 * array: calls that overlap in time on one device (other streams, or graph
 * replays beside eager calls) race and give wrong results. Added in ABI 1.03.
 */
int mgi_paged_decode_noalloc(void* out, const int64_t* out_strides, /* [3] */
                             const void* q, const int64_t* q_strides, /* [3] */
                             const void* k_pool, const void* v_pool,
                             const int64_t* k_pool_strides, /* [5] */
                             const int64_t* v_pool_strides, /* [5] */
                             int dtype,
                             const void* block_tables, const int64_t* bt_strides, /* [2] */
                             int bt_itype,
                             const void* context_lens, int64_t cl_stride, int cl_itype,
                             int64_t B, int64_t H, int64_t D, int64_t S, int64_t N,
                             int64_t M, int64_t L, int64_t layer_idx,
                             float scale, int64_t split_tokens,
                             void* stream);

/* Workspace bytes mgi_paged_decode needs for these sizes (0 if none). */
size_t mgi_paged_decode_workspace_bytes(int64_t B, int64_t H, int64_t D,
                                        int64_t S, int64_t M,
                                        int64_t split_tokens);

/* The partition size (tokens) mgi_paged_decode uses for these sizes when it
 * splits contexts into partitions. */
int64_t mgi_paged_decode_split_tokens(int64_t B, int64_t H, int64_t D,
                                      int64_t S, int64_t M,
                                      int64_t split_tokens);

/* Wavefronts per group of heads of the even split mgi_paged_decode uses for
 * these sizes on the current device, or 0 when it splits into partitions
 * (or does not split). No counterpart in the reference: it reports the
 * split, as mgi_paged_decode_split_tokens does. */
int64_t mgi_paged_decode_balanced_waves(int64_t B, int64_t H, int64_t D,
                                        int64_t S, int64_t M,
                                        int64_t split_tokens);

/*
 * Paged prefill attention of one chunk of one sequence.
 * Replaces the per-token prefill loop of
 * KVCacheCausalSelfAttention.forward_prefill_chunk
 * (minivllm/attention.py:269-299, paged_attention_online per query) and the
 * prefix-aware gather + SDPA of mode sdpa_v2 (minivllm/attention.py:229-267).
 *
 * The chunk holds T query rows at absolute positions start_pos .. start_pos+T-1;
 * its own K/V rows must already be in the pool (mgi_kv_append on the same
 * stream). For t < T, h < H:
 *   out[t,h,:] = sum_j softmax_j(scale * q[t,h,:] . K[j,h,:]) * V[j,h,:]
 * over the logical tokens j = 0 .. start_pos + t, where token j lives in
 * physical block block_table[j / S] at offset j % S of layer layer_idx.
 * block_table must hold n_blocks >= ceil((start_pos + T) / S) entries; only
 * those are read. An entry outside [0, N) is treated as a fully masked block.
 * q, out and the pool share one dtype; arithmetic is fp32 (bf16 inputs run
 * on the bf16 matrix cores with P rounded to bf16 for the PV product).
 * Layouts: q, out [T, H, D] (any strides); block_table [n_blocks] with
 * element stride bt_stride.
 * A short chunk after a long prefix (2-byte types, head_dim a multiple of
 * 8, too few query tiles to fill the GPU, and a cost model that says it
 * pays) has its keys split over several workgroups per query tile and the
 * partials merged in a second pass; workspace must then hold
 * mgi_paged_prefill_workspace_bytes(...) bytes for the same (start_pos, T,
 * H, D, dtype), and it may be NULL when that is 0. Its contents need no
 * initialisation; calls that overlap in time need separate workspaces.
 * MINIVLLM_HIP_PREFILL_SPLIT_KEYS (read on every call, by both functions)
 * turns the split off (-1) or forces that many keys per partition (> 0).
 * (ABI 1.02 added workspace, workspace_bytes.)
 */
int mgi_paged_prefill(void* out, const int64_t* out_strides, /* [3] */
                      const void* q, const int64_t* q_strides, /* [3] */
                      const void* k_pool, const void* v_pool,
                      const int64_t* k_pool_strides, /* [5] */
                      const int64_t* v_pool_strides, /* [5] */
                      int dtype,
                      const void* block_table, int64_t bt_stride, int bt_itype,
                      int64_t n_blocks, int64_t start_pos, int64_t T,
                      int64_t H, int64_t D, int64_t S, int64_t N,
                      int64_t L, int64_t layer_idx, float scale,
                      void* workspace, size_t workspace_bytes,
                      void* stream);

/* Workspace bytes mgi_paged_prefill needs for these sizes on the current
 * device (0 if it does not split the keys). No counterpart in the
 * reference: it sizes the workspace of the split, as
 * mgi_paged_decode_workspace_bytes does for decode. */
size_t mgi_paged_prefill_workspace_bytes(int64_t start_pos, int64_t T,
                                         int64_t H, int64_t D, int dtype);

#ifdef __cplusplus
}
#endif

#endif /* MINIVLLM_HIP_H */
