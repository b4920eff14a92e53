// mgi_internal.h -- argument blocks passed by value to the kernels, and the
// host-side launchers the C ABI (capi.hip) dispatches to.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace mgi {

// Paged decode attention. Pool pointers already point at layer layer_idx.
// All strides are in elements.
struct DecodeArgs {
  void* out;
  int64_t o_sb, o_sh, o_sd;
  const void* q;
  int64_t q_sb, q_sh, q_sd;
  const void* k;
  const void* v;
  int64_t k_sn, k_ss, k_sh, k_sd;
  int64_t v_sn, v_ss, v_sh, v_sd;
  const void* bt;
  int64_t bt_sb, bt_sm;
  const void* cl;      // null: row b's context length is ctx_base + b + 1
  int64_t cl_s;
  int64_t ctx_base;
  int bt_i64, cl_i64;
  int B, H, D, S, M;
  int64_t N;
  float scale_log2;   // softmax scale * log2(e): scores live in the log2 domain
  int part_tokens;    // partition mode: tokens per context partition (multiple of S)
  int max_parts;      // partials per (sequence, head) the workspace holds
  int bal_waves;      // > 0: balanced mode with this many waves per head group
  int bal_min_blocks; // balanced mode: least blocks per claim
  int bal_tier1_16ths;// balanced mode: share of each segment in its wave's own claim (16ths)
  int bal_tier2;      // balanced mode: ticket claims per segment, at most (0: none)
  int bal_claims;     // balanced mode: bal_waves * (1 + bal_tier2), partial slot pairs per head
  int merge_waves;    // wavefronts per workgroup of paged_decode_merge (1, 2, 4 or 8)
  float* ws_acc;      // [B, H, max_parts, D] unnormalised partial outputs
  float2* ws_ml;      // [B, H, max_parts]    partial (max, sum), log2 domain
  int* ws_cinc;       // balanced mode: [B] inclusive prefix sums of blocks per sequence
  int* ws_ticket;     // balanced mode: one ticket counter per head group
  // Fused KV append (fast path only; kw == nullptr: none). Row b of kn / vn
  // ([B, H, D], head dim contiguous, rows 16-byte aligned) goes to pool slot
  // slots[b] (skipped when outside [0, N*S)), written by each head group's
  // wavefront that streams sequence b's last block, before it reads that
  // block; rows of sequences with no blocks by a wavefront of their own.
  void* kw;           // the pool at layer layer_idx (k, v), writable
  void* vw;
  const void* kn;
  const void* vn;
  int64_t kn_sb, kn_sh, vn_sb, vn_sh;
  const void* slots;
  int64_t sl_s;
  int sl_i64;
};

// KV append / scatter. Pool pointers already point at layer layer_idx.
struct AppendArgs {
  void* kp;
  void* vp;
  int64_t k_sn, k_ss, k_sh, k_sd;
  int64_t v_sn, v_ss, v_sh, v_sd;
  const void* kn;
  const void* vn;
  int64_t kn_st, kn_sh, kn_sd;
  int64_t vn_st, vn_sh, vn_sd;
  const void* slots;
  int64_t sl_s;
  int sl_i64;
  int T, H, D, S;
  int64_t N;
};

// Paged prefill attention of one chunk: query row i (absolute position
// start + i) attends keys 0 .. start + i through one block-table row. Pool
// pointers already point at layer layer_idx; strides are in elements and the
// head dim is contiguous everywhere.
struct PrefillArgs {
  void* out;
  int64_t o_st, o_sh;
  const void* q;
  int64_t q_st, q_sh;
  const void* k;
  const void* v;
  int64_t k_sn, k_ss, k_sh;
  int64_t v_sn, v_ss, v_sh;
  const void* bt;
  int64_t bt_s;
  int bt_i64;
  int start, T, H, D, S;
  int s_shift;        // log2(S) when S is a power of two, else -1
  int64_t N;
  float scale_log2;   // softmax scale * log2(e)
  int pair_round;     // > 0: workgroups per XCD in one slot round (see the kernel's grid mapping)
  int cus;            // compute units of the device (set by the caller)
  int part_keys;      // > 0: keys per partition (a multiple of 64) when the keys are split
  int max_parts;      // split keys: partitions per row the workspace holds
  float* ws_acc;      // split keys: [T, H, max_parts, D] unnormalised partial outputs
  float2* ws_ml;      // split keys: [T, H, max_parts] partial (max, sum), log2 domain
};

// Largest batch of the fast decode kernel's balanced mode (its per-wave
// prefix sums of blocks per sequence live in LDS).
constexpr int kBalMaxB = 4096;

enum class DecodePath { kFast, kGeneric };

// Paged decode: how a call will run (decided from dtype, shapes, strides and
// pointer alignment) and the launchers.
struct DecodePlan {
  DecodePath path;
  int lanes_per_head;   // fast path: lanes that share one head row
  int tokens_per_step;  // fast path: tokens loaded per inner step
  bool full_lanes;      // fast path: every lane maps to a valid (head, d)
};

hipError_t launch_paged_decode(const DecodeArgs& a, int dtype, const DecodePlan& plan,
                               hipStream_t stream);

// Paged prefill on the matrix cores. `dp` is the padded head dim returned by
// prefill_head_dim_bucket (0: no MFMA variant); `waves` is 2 or 4; `qpw` is
// the number of 16-row query blocks per wavefront (1).
int prefill_head_dim_bucket(int two_byte, int D);
hipError_t launch_paged_prefill(const PrefillArgs& a, int dtype, int dp, int waves, int qpw,
                                hipStream_t stream);

// paged_decode_merge alone (partition mode), for partials another kernel wrote
// in its layout; `lanes_per_head` as in DecodePlan.
hipError_t launch_paged_merge(const DecodeArgs& a, int dtype, int lanes_per_head, hipStream_t stream);

// KV append launchers. `vector_path` copies 16-byte chunks (same dtype,
// contiguous aligned rows); otherwise an element loop converts dtypes.
hipError_t launch_kv_append(const AppendArgs& a, int pool_dtype, int new_dtype,
                            bool vector_path, hipStream_t stream);

}  // namespace mgi
