// kv_append.hip -- KV append / scatter for gfx950.
//
// Semantics of the decode KV write in
// KVCacheCausalSelfAttention.forward_decode_batch (minivllm/attention.py:370-392):
//   blk = slot // S, off = slot % S, pool.k[layer, blk, off] = k[t] (same for v)
// with one deliberate difference: a negative slot marks a padding row that is
// skipped (the reference would wrap it to the last block), and a slot past the
// pool is skipped as well, so no byte outside the named slots is written.
//
// Grid: (T rows, 2) -- y selects K or V. One workgroup copies one H*D row.
// The vector path moves 16-byte chunks (bit-exact, same dtype, contiguous
// aligned rows); the element path handles any strides and converts dtypes.
#include <type_traits>

#include "mgi_common.h"
#include "mgi_internal.h"
#include "minivllm_hip.h"

namespace mgi {

constexpr int kAppendThreads = 256;

__device__ __forceinline__ bool append_target(const AppendArgs& a, int t, int64_t* blk,
                                              int64_t* off) {
  const int64_t slot = load_index(a.slots, a.sl_i64, (int64_t)t * a.sl_s);
  if (slot < 0 || slot >= a.N * (int64_t)a.S) return false;
  *blk = slot / a.S;
  *off = slot - *blk * a.S;
  return true;
}

// Same dtype, pool row and source row each contiguous over (H, D) and
// 16-byte aligned: copy row_bytes / 16 chunks.
__global__ void __launch_bounds__(kAppendThreads)
kv_append_vec16(const AppendArgs a, int elem_bytes) {
  const int t = (int)blockIdx.x;
  const bool is_v = blockIdx.y != 0;
  int64_t blk, off;
  if (!append_target(a, t, &blk, &off)) return;
  const int64_t chunks = (int64_t)a.H * a.D * elem_bytes / 16;
  const char* src = reinterpret_cast<const char*>(is_v ? a.vn : a.kn) +
                    (int64_t)t * (is_v ? a.vn_st : a.kn_st) * elem_bytes;
  char* dst = reinterpret_cast<char*>(is_v ? a.vp : a.kp) +
              (blk * (is_v ? a.v_sn : a.k_sn) + off * (is_v ? a.v_ss : a.k_ss)) * elem_bytes;
  const uint4* s4 = reinterpret_cast<const uint4*>(src);
  uint4* d4 = reinterpret_cast<uint4*>(dst);
  for (int64_t c = threadIdx.x; c < chunks; c += kAppendThreads) d4[c] = s4[c];
}

template <typename TS, typename TD>
__global__ void __launch_bounds__(kAppendThreads)
kv_append_elem(const AppendArgs a) {
  const int t = (int)blockIdx.x;
  const bool is_v = blockIdx.y != 0;
  int64_t blk, off;
  if (!append_target(a, t, &blk, &off)) return;
  const TS* src = reinterpret_cast<const TS*>(is_v ? a.vn : a.kn) +
                  (int64_t)t * (is_v ? a.vn_st : a.kn_st);
  const int64_t s_sh = is_v ? a.vn_sh : a.kn_sh, s_sd = is_v ? a.vn_sd : a.kn_sd;
  TD* dst = reinterpret_cast<TD*>(is_v ? a.vp : a.kp) +
            blk * (is_v ? a.v_sn : a.k_sn) + off * (is_v ? a.v_ss : a.k_ss);
  const int64_t d_sh = is_v ? a.v_sh : a.k_sh, d_sd = is_v ? a.v_sd : a.k_sd;
  const int64_t n = (int64_t)a.H * a.D;
  for (int64_t i = threadIdx.x; i < n; i += kAppendThreads) {
    const int64_t h = i / a.D, d = i - h * a.D;
    const TS x = src[h * s_sh + d * s_sd];
    TD* y = dst + h * d_sh + d * d_sd;
    if constexpr (std::is_same_v<TS, TD>) {
      *y = x;  // raw copy: bit-exact, NaN payloads included
    } else {
      Elem<TD>::store(y, Elem<TS>::load(&x));
    }
  }
}

template <typename TS, typename TD>
static const void* elem_kernel() {
  return reinterpret_cast<const void*>(&kv_append_elem<TS, TD>);
}

hipError_t launch_kv_append(const AppendArgs& a, int pool_dtype, int new_dtype, bool vector_path,
                            hipStream_t stream) {
  if (a.T <= 0) return hipSuccess;
  const dim3 grid((unsigned)a.T, 2u), block(kAppendThreads);
  if (vector_path) {
    int eb = pool_dtype == MGI_F32 ? 4 : 2;
    void* args[] = {const_cast<AppendArgs*>(&a), &eb};
    return hipLaunchKernel(reinterpret_cast<const void*>(&kv_append_vec16), grid, block, args, 0,
                           stream);
  }
  const void* fn = nullptr;
  if (pool_dtype == new_dtype) {
    fn = pool_dtype == MGI_F32    ? elem_kernel<float, float>()
         : pool_dtype == MGI_BF16 ? elem_kernel<bf16_t, bf16_t>()
                                  : elem_kernel<f16_t, f16_t>();
  } else if (new_dtype == MGI_F32 && pool_dtype == MGI_BF16) {
    fn = elem_kernel<float, bf16_t>();
  } else if (new_dtype == MGI_F32 && pool_dtype == MGI_F16) {
    fn = elem_kernel<float, f16_t>();
  } else if (new_dtype == MGI_BF16 && pool_dtype == MGI_F32) {
    fn = elem_kernel<bf16_t, float>();
  } else if (new_dtype == MGI_F16 && pool_dtype == MGI_F32) {
    fn = elem_kernel<f16_t, float>();
  } else {
    return hipErrorInvalidValue;
  }
  void* args[] = {const_cast<AppendArgs*>(&a)};
  return hipLaunchKernel(fn, grid, block, args, 0, stream);
}

}  // namespace mgi
