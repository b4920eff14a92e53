// torch_ops.cpp -- the PyTorch-side binding of libminivllm_hip.so for the
// eager Python path (module minivllm._native._hip_ops).
//
// Each function validates its tensors exactly as the Python wrappers in
// minivllm/hip_paged_decode.py do (same exception types and messages; the
// Python contract follows paged_attention_batch_triton_v0,
// minivllm/triton_paged_decode.py:109-144), takes data pointers and strides
// straight from the tensors, allocates outputs and workspaces through
// PyTorch's caching allocator, and calls the C ABI declared in
// include/minivllm_hip.h on the current HIP stream. It replaces the ctypes
// marshalling of 20-30 arguments per call; the kernels and their launch
// decisions are the library's, unchanged. Nothing here computes attention.
#include <ATen/hip/HIPContext.h>
#include <torch/extension.h>

#include <cmath>
#include <string>

#include "minivllm_hip.h"

namespace {

void check_status(int status) {
  if (status == MGI_OK) return;
  const char* m = mgi_last_error();
  const std::string msg = m ? m : "";
  if (status == MGI_EINVAL || status == MGI_EUNSUPPORTED) throw pybind11::value_error(msg);
  throw std::runtime_error("libminivllm_hip error " + std::to_string(status) + ": " + msg);
}

[[noreturn]] void value_error(const char* msg) { throw pybind11::value_error(msg); }

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return MGI_F32;
    case at::kBFloat16: return MGI_BF16;
    case at::kHalf: return MGI_F16;
    default: return -1;
  }
}

int index_code(at::ScalarType t) {
  switch (t) {
    case at::kInt: return MGI_I32;
    case at::kLong: return MGI_I64;
    default: return -1;
  }
}

void* stream_of(const at::Tensor& t) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_pool(const at::Tensor& kp, const at::Tensor& vp) {
  if (kp.dim() != 5 || vp.sizes() != kp.sizes()) value_error("KV tensors must have matching [L,P,S,H,D] shape");
}

// kv_append(k_pool, v_pool, layer_idx, k, v, slot_mapping): rows k[t], v[t]
// into pool slots slot_mapping[t] (negative slots skipped).
void kv_append(const at::Tensor& kp, const at::Tensor& vp, int64_t layer_idx, const at::Tensor& k,
               const at::Tensor& v, const at::Tensor& slots) {
  if (!kp.is_cuda()) value_error("KV pool must be on a GPU device for the HIP backend");
  if (k.dim() != 3 || v.sizes() != k.sizes()) value_error("k and v must have matching shape [T,H,D]");
  check_pool(kp, vp);
  const int64_t T = k.size(0), L = kp.size(0), N = kp.size(1), S = kp.size(2), H = kp.size(3), D = kp.size(4);
  if (S <= 0) value_error("block_size must be positive");
  if (k.size(1) != H || k.size(2) != D) value_error("k/v head dimensions do not match the KV pool");
  const int pd = dtype_code(kp.scalar_type());
  if (pd < 0 || vp.scalar_type() != kp.scalar_type()) value_error("KV pool must be float32, bfloat16 or float16");
  const int nd = dtype_code(k.scalar_type());
  if (nd < 0 || v.scalar_type() != k.scalar_type()) value_error("k and v must share a float dtype");
  if (slots.dim() != 1 || slots.size(0) != T) value_error("slot_mapping must have shape [T]");
  const int st = index_code(slots.scalar_type());
  if (st < 0) value_error("slot_mapping must contain integer slots");
  if (layer_idx < 0 || layer_idx >= L) value_error("layer_idx outside KV pool");
  const auto dev = kp.device();
  if (vp.device() != dev || k.device() != dev || v.device() != dev || slots.device() != dev)
    value_error("all inputs must reside on same GPU device");
  if (T == 0) return;
  check_status(mgi_kv_append(kp.data_ptr(), vp.data_ptr(), kp.strides().data(), vp.strides().data(), pd,
                             k.data_ptr(), v.data_ptr(), k.strides().data(), v.strides().data(), nd,
                             slots.data_ptr(), slots.stride(0), st, T, H, D, S, N, L, layer_idx, stream_of(kp)));
}

// Checks of paged_decode's arguments (the Triton v0 backend's order and
// messages); returns the block-table width M.
int64_t check_decode(const at::Tensor& q, const at::Tensor& kp, const at::Tensor& vp, const at::Tensor& bt,
                     const at::Tensor& cl, int64_t layer_idx) {
  if (!q.is_cuda()) value_error("q must be on a GPU device for the HIP backend");
  if (q.dim() != 3) value_error("q must have shape [B,H,D]");
  const int64_t b = q.size(0), h = q.size(1), d = q.size(2);
  if (b == 0 || h == 0 || d == 0) value_error("q dimensions must be nonzero");
  if (d > 512) value_error("HIP backend supports head_dim <= 512");
  const int qd = dtype_code(q.scalar_type());
  if (qd < 0) value_error("q must be float32, bfloat16 or float16");
  if (kp.scalar_type() != q.scalar_type() || vp.scalar_type() != q.scalar_type())
    value_error("KV pool dtype must match q dtype");
  check_pool(kp, vp);
  const int64_t L = kp.size(0), S = kp.size(2);
  if (S <= 0) value_error("block_size must be positive");
  if (kp.size(3) != h || kp.size(4) != d) value_error("KV head dimensions or block size do not match q");
  if (bt.dim() != 2 || bt.size(0) != b) value_error("block_tables must have shape [B,M]");
  if (cl.dim() != 1 || cl.size(0) != b) value_error("context_lengths must have shape [B]");
  if (index_code(bt.scalar_type()) < 0) value_error("block_tables must contain integer indices");
  if (index_code(cl.scalar_type()) < 0) value_error("context_lengths must be integer");
  if (layer_idx < 0 || layer_idx >= L) value_error("layer_idx outside KV pool");
  const auto dev = q.device();
  if (kp.device() != dev || vp.device() != dev || bt.device() != dev || cl.device() != dev)
    value_error("all inputs must reside on same GPU device");
  const int64_t M = bt.size(1);
  if (M < 1) value_error("block_tables need at least one block column");
  return M;
}

// paged_decode(q, k_pool, v_pool, block_tables, context_lengths, layer_idx,
// split_tokens) -> [B, H, D] attention output of q's dtype.
at::Tensor paged_decode(const at::Tensor& q, const at::Tensor& kp, const at::Tensor& vp, const at::Tensor& bt,
                        const at::Tensor& cl, int64_t layer_idx, int64_t split_tokens) {
  const int64_t M = check_decode(q, kp, vp, bt, cl, layer_idx);
  const int64_t b = q.size(0), h = q.size(1), d = q.size(2), L = kp.size(0), N = kp.size(1), S = kp.size(2);
  at::Tensor out = at::empty({b, h, d}, q.options());
  const size_t ws_bytes = mgi_paged_decode_workspace_bytes(b, h, d, S, M, split_tokens);
  at::Tensor ws;
  if (ws_bytes) ws = at::empty({(int64_t)ws_bytes}, q.options().dtype(at::kByte));
  check_status(mgi_paged_decode(out.data_ptr(), out.strides().data(), q.data_ptr(), q.strides().data(),
                                kp.data_ptr(), vp.data_ptr(), kp.strides().data(), vp.strides().data(),
                                dtype_code(q.scalar_type()), bt.data_ptr(), bt.strides().data(),
                                index_code(bt.scalar_type()), cl.data_ptr(), cl.stride(0),
                                index_code(cl.scalar_type()), b, h, d, S, N, M, L, layer_idx,
                                (float)(1.0 / std::sqrt((double)d)), split_tokens,
                                ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, stream_of(q)));
  return out;
}

// paged_decode_append(q, k_pool, v_pool, block_tables, context_lengths,
// layer_idx, k, v, slot_mapping, split_tokens) -> [B, H, D]: kv_append of
// the B rows k[b], v[b] into slot_mapping[b], then paged_decode, as one call
// (one launch fewer where the library fuses them).
at::Tensor paged_decode_append(const at::Tensor& q, const at::Tensor& kp, const at::Tensor& vp,
                               const at::Tensor& bt, const at::Tensor& cl, int64_t layer_idx, const at::Tensor& k,
                               const at::Tensor& v, const at::Tensor& slots, int64_t split_tokens) {
  const int64_t M = check_decode(q, kp, vp, bt, cl, layer_idx);
  const int64_t b = q.size(0), h = q.size(1), d = q.size(2), L = kp.size(0), N = kp.size(1), S = kp.size(2);
  if (k.dim() != 3 || v.sizes() != k.sizes()) value_error("k and v must have matching shape [T,H,D]");
  if (k.size(0) != b) value_error("k and v must hold one row per sequence");
  if (k.size(1) != h || k.size(2) != d) value_error("k/v head dimensions do not match the KV pool");
  const int nd = dtype_code(k.scalar_type());
  if (nd < 0 || v.scalar_type() != k.scalar_type()) value_error("k and v must share a float dtype");
  if (slots.dim() != 1 || slots.size(0) != b) value_error("slot_mapping must have shape [B]");
  const int st = index_code(slots.scalar_type());
  if (st < 0) value_error("slot_mapping must contain integer slots");
  const auto dev = q.device();
  if (k.device() != dev || v.device() != dev || slots.device() != dev)
    value_error("all inputs must reside on same GPU device");
  at::Tensor out = at::empty({b, h, d}, q.options());
  const size_t ws_bytes = mgi_paged_decode_workspace_bytes(b, h, d, S, M, split_tokens);
  at::Tensor ws;
  if (ws_bytes) ws = at::empty({(int64_t)ws_bytes}, q.options().dtype(at::kByte));
  check_status(mgi_paged_decode_append(
      out.data_ptr(), out.strides().data(), q.data_ptr(), q.strides().data(), kp.data_ptr(), vp.data_ptr(),
      kp.strides().data(), vp.strides().data(), dtype_code(q.scalar_type()), k.data_ptr(), v.data_ptr(),
      k.strides().data(), v.strides().data(), nd, slots.data_ptr(), slots.stride(0), st, bt.data_ptr(),
      bt.strides().data(), index_code(bt.scalar_type()), cl.data_ptr(), cl.stride(0), index_code(cl.scalar_type()),
      b, h, d, S, N, M, L, layer_idx, (float)(1.0 / std::sqrt((double)d)), split_tokens,
      ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, stream_of(q)));
  return out;
}

// paged_prefill(q, k_pool, v_pool, block_table, start_pos, layer_idx) ->
// [T, H, D] causal attention of the chunk's rows over the pool.
at::Tensor paged_prefill(const at::Tensor& q, const at::Tensor& kp, const at::Tensor& vp, const at::Tensor& bt,
                         int64_t start_pos, int64_t layer_idx) {
  if (!q.is_cuda()) value_error("q must be on a GPU device for the HIP backend");
  if (q.dim() != 3) value_error("q must have shape [T,H,D]");
  const int64_t t = q.size(0), h = q.size(1), d = q.size(2);
  if (h == 0 || d == 0) value_error("q dimensions must be nonzero");
  if (d > 512) value_error("HIP backend supports head_dim <= 512");
  const int qd = dtype_code(q.scalar_type());
  if (qd < 0) value_error("q must be float32, bfloat16 or float16");
  if (kp.scalar_type() != q.scalar_type() || vp.scalar_type() != q.scalar_type())
    value_error("KV pool dtype must match q dtype");
  check_pool(kp, vp);
  const int64_t L = kp.size(0), N = kp.size(1), S = kp.size(2);
  if (S <= 0) value_error("block_size must be positive");
  if (kp.size(3) != h || kp.size(4) != d) value_error("KV head dimensions do not match q");
  const int bti = index_code(bt.scalar_type());
  if (bt.dim() != 1 || bti < 0) value_error("block_table must be a 1-D integer tensor");
  if (start_pos < 0) value_error("start_pos must be non-negative");
  if (bt.size(0) < (start_pos + t + S - 1) / S) value_error("block_table shorter than ceil((start_pos + T) / S)");
  if (layer_idx < 0 || layer_idx >= L) value_error("layer_idx outside KV pool");
  const auto dev = q.device();
  if (kp.device() != dev || vp.device() != dev || bt.device() != dev)
    value_error("all inputs must reside on same GPU device");
  at::Tensor out = at::empty({t, h, d}, q.options());
  if (t == 0) return out;
  const size_t ws_bytes = mgi_paged_prefill_workspace_bytes(start_pos, t, h, d, qd);
  at::Tensor ws;
  if (ws_bytes) ws = at::empty({(int64_t)ws_bytes}, q.options().dtype(at::kByte));
  check_status(mgi_paged_prefill(out.data_ptr(), out.strides().data(), q.data_ptr(), q.strides().data(),
                                 kp.data_ptr(), vp.data_ptr(), kp.strides().data(), vp.strides().data(), qd,
                                 bt.data_ptr(), bt.stride(0), bti, bt.size(0), start_pos, t, h, d, S, N, L,
                                 layer_idx, (float)(1.0 / std::sqrt((double)d)), ws_bytes ? ws.data_ptr() : nullptr,
                                 ws_bytes, stream_of(q)));
  return out;
}

}  // namespace

PYBIND11_MODULE(_hip_ops, m) {
  m.doc() = "PyTorch binding of libminivllm_hip.so (kv_append, paged_decode, paged_decode_append, paged_prefill)";
  m.def("kv_append", &kv_append);
  m.def("paged_decode", &paged_decode);
  m.def("paged_decode_append", &paged_decode_append);
  m.def("paged_prefill", &paged_prefill);
}
