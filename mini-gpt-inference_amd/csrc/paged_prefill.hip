// paged_prefill.hip -- causal attention of one prefill chunk over the paged
// KV pool, on the matrix cores of gfx950.
//
// Query row i of the chunk sits at absolute position start + i and attends
// keys 0 .. start + i of its sequence, all read from the pool through the
// sequence's block table (the chunk's own K/V rows are appended to the pool
// first, on the same stream). This is what the reference computes per token
// (minivllm/attention.py:269-299, paged_attention_online) and with the
// gathered-prefix SDPA of mode sdpa_v2 (minivllm/attention.py:229-267).
//
// Work split: one workgroup per (query tile, head); each wavefront owns 16
// query rows. Keys stream through LDS in tiles of 64: K row-major, V
// transposed. Each wave computes S^T = K Q^T and O^T += V^T P^T with
// 16x16 MFMA tiles, so a lane's accumulator column is one query row: the
// online-softmax state (max, sum) is per lane and P needs no transpose.
//
// Numerics: fp32 accumulation and softmax in the log2 domain; bf16 inputs
// use v_mfma_f32_16x16x32_bf16 with P rounded to bf16 for the PV product,
// fp32 inputs use v_mfma_f32_16x16x4_f32 (full fp32 products).
#include "mgi_common.h"
#include "mgi_internal.h"

namespace mgi {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTileKeys = 64;  // keys per LDS tile

template <typename T> struct PF;
template <> struct PF<bf16_t> {
  static constexpr int kChunk = 8;  // elements per 16-byte chunk
  static constexpr int kKPad = 8;   // K tile row padding (elements): conflict-free b128 reads
  static constexpr int kVPad = 8;   // V^T row padding: conflict-free b64 reads and writes
};
template <> struct PF<float> {
  static constexpr int kChunk = 4;
  static constexpr int kKPad = 4;
  static constexpr int kVPad = 4;
};

__device__ __forceinline__ float shfl_xor32(float x) { return __shfl_xor(x, 32, 64); }

// Reduction over the four lanes l, l^16, l^32, l^48 that hold one query's keys.
__device__ __forceinline__ float cross_group_max(float x) {
  x = fmaxf(x, swizzle_xor16(x));
  return fmaxf(x, shfl_xor32(x));
}
__device__ __forceinline__ float cross_group_sum(float x) {
  x += swizzle_xor16(x);
  return x + shfl_xor32(x);
}

// Block-table slot of key `key` of the workgroup: (physical block, offset),
// or (-1, 0) for keys past the chunk or invalid table entries.
__device__ __forceinline__ int2 key_slot(const PrefillArgs& a, int key, int kv_end) {
  if (key >= kv_end) return make_int2(-1, 0);
  int blk, off;
  if (a.s_shift >= 0) {
    blk = key >> a.s_shift;
    off = key & (a.S - 1);
  } else {
    blk = key / a.S;
    off = key - blk * a.S;
  }
  const int64_t phys = load_index(a.bt, a.bt_i64, (int64_t)blk * a.bt_s);
  if (phys < 0 || phys >= a.N) return make_int2(-1, 0);
  return make_int2((int)phys, off);
}

template <typename T, int DP, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void paged_prefill_mfma(const PrefillArgs a) {
  using E = PF<T>;
  constexpr int CH = E::kChunk;
  constexpr int CPR = DP / CH;                 // 16-byte chunks per key row
  constexpr int KROW = DP + E::kKPad;          // K tile row stride (elements)
  constexpr int VROW = kTileKeys + E::kVPad;   // V^T tile row stride (elements)
  constexpr int NT = 64 * WAVES;
  constexpr int ITEMS = 16 * CPR;              // (4-key group, chunk) pairs per tile
  constexpr int IPT = (ITEMS + NT - 1) / NT;
  constexpr int QB = 16 * WAVES;               // query rows per workgroup
  constexpr bool kBF16 = sizeof(T) == 2;
  constexpr int NQF = kBF16 ? DP / 32 : DP / 16;   // Q fragments (16 bytes each)
  constexpr int NDB = DP / 16;                     // 16-wide head-dim blocks of O^T

  __shared__ __align__(16) T k_lds[kTileKeys * KROW];
  __shared__ __align__(16) T vt_lds[DP * VROW];
  __shared__ int2 slots[2][kTileKeys];

  const int qt = (int)gridDim.x - 1 - (int)blockIdx.x;  // longest query tiles first
  const int h = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 15, g = lane >> 4;
  const int qw0 = qt * QB + wave * 16;
  const int qi = qw0 + col;
  const bool q_ok = qi < a.T;
  const int qpos = a.start + (q_ok ? qi : a.T - 1);
  const int kv_end = a.start + min(a.T, (qt + 1) * QB);
  const bool wave_active = qw0 < a.T;
  const int wave_last = a.start + min(a.T, qw0 + 16) - 1;
  const int ntiles = (kv_end + kTileKeys - 1) / kTileKeys;

  // ---- this lane's query fragments (zero past the chunk or past D)
  uint4 qf[NQF];
  {
    const T* qrow = reinterpret_cast<const T*>(a.q) + (int64_t)(q_ok ? qi : 0) * a.q_st +
                    (int64_t)h * a.q_sh;
#pragma unroll
    for (int f = 0; f < NQF; ++f) {
      const int d = kBF16 ? 32 * f + 8 * g : 16 * f + 4 * g;
      qf[f] = (q_ok && d < a.D) ? *reinterpret_cast<const uint4*>(qrow + d) : make_uint4(0, 0, 0, 0);
    }
  }

  const T* kb_ = reinterpret_cast<const T*>(a.k) + (int64_t)h * a.k_sh;
  const T* vb_ = reinterpret_cast<const T*>(a.v) + (int64_t)h * a.v_sh;

  // Staging registers: item j of this thread covers 4 keys x one chunk, for K
  // (keys vary slowest: lanes sweep the head dim) and V (lanes sweep keys).
  uint4 kr[IPT][4], vr[IPT][4];
  auto load_tile = [&](int buf) {
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      const int it = tid + NT * j;
      const bool in = (ITEMS % NT == 0) || it < ITEMS;
      const int kq_k = it / CPR, dc_k = it % CPR;
      const int kq_v = it % 16, dc_v = it / 16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int2 sk = slots[buf][4 * kq_k + r];
        const int2 sv = slots[buf][4 * kq_v + r];
        const bool okk = in && sk.x >= 0 && dc_k * CH < a.D;
        const bool okv = in && sv.x >= 0 && dc_v * CH < a.D;
        kr[j][r] = okk ? *reinterpret_cast<const uint4*>(kb_ + (int64_t)sk.x * a.k_sn +
                                                         (int64_t)sk.y * a.k_ss + dc_k * CH)
                       : make_uint4(0, 0, 0, 0);
        vr[j][r] = okv ? *reinterpret_cast<const uint4*>(vb_ + (int64_t)sv.x * a.v_sn +
                                                         (int64_t)sv.y * a.v_ss + dc_v * CH)
                       : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      const int it = tid + NT * j;
      if (!((ITEMS % NT == 0) || it < ITEMS)) continue;
      const int kq_k = it / CPR, dc_k = it % CPR;
      const int kq_v = it % 16, dc_v = it / 16;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<uint4*>(&k_lds[(4 * kq_k + r) * KROW + dc_k * CH]) = kr[j][r];
      if constexpr (kBF16) {
        // 8 head dims x 4 keys -> eight 4-key rows of V^T.
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int w = e >> 1, sh = (e & 1) * 16;
          auto word = [&](const uint4& x) {
            const uint32_t v = w == 0 ? x.x : w == 1 ? x.y : w == 2 ? x.z : x.w;
            return (v >> sh) & 0xffffu;
          };
          uint2 pk;
          pk.x = word(vr[j][0]) | (word(vr[j][1]) << 16);
          pk.y = word(vr[j][2]) | (word(vr[j][3]) << 16);
          *reinterpret_cast<uint2*>(&vt_lds[(8 * dc_v + e) * VROW + 4 * kq_v]) = pk;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          auto word = [&](const uint4& x) { return e == 0 ? x.x : e == 1 ? x.y : e == 2 ? x.z : x.w; };
          uint4 pk = make_uint4(word(vr[j][0]), word(vr[j][1]), word(vr[j][2]), word(vr[j][3]));
          *reinterpret_cast<uint4*>(&vt_lds[(4 * dc_v + e) * VROW + 4 * kq_v]) = pk;
        }
      }
    }
  };

  f32x4_t oacc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) oacc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_part = 0.f;

  // Prologue: slots of tile 0 (and a prefetch of tile 1), then tile 0's data.
  int2 slot_next = make_int2(-1, 0);
  if (tid < kTileKeys) {
    slots[0][tid] = key_slot(a, tid, kv_end);
    if (ntiles > 1) slot_next = key_slot(a, kTileKeys + tid, kv_end);
  }
  __syncthreads();
  load_tile(0);

  for (int t = 0; t < ntiles; ++t) {
    const int kt0 = t * kTileKeys;
    if (tid < kTileKeys) {
      slots[(t + 1) & 1][tid] = slot_next;
      if (t + 2 < ntiles) slot_next = key_slot(a, (t + 2) * kTileKeys + tid, kv_end);
    }
    store_tile();
    __syncthreads();
    if (t + 1 < ntiles) load_tile((t + 1) & 1);

    if (wave_active && kt0 <= wave_last) {
      // ---- S^T tile: lane holds keys kt0 + 16*kb + 4*g + i of query column `col`
      f32x4_t s[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        s[kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        const T* krow = &k_lds[(16 * kb + col) * KROW];
        if constexpr (kBF16) {
#pragma unroll
          for (int f = 0; f < NQF; ++f) {
            const uint4 kv = *reinterpret_cast<const uint4*>(krow + 32 * f + 8 * g);
            s[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kv),
                                                            __builtin_bit_cast(bf16x8_t, qf[f]),
                                                            s[kb], 0, 0, 0);
          }
        } else {
#pragma unroll
          for (int f = 0; f < NQF; ++f) {
            const float4 kv = *reinterpret_cast<const float4*>(krow + 16 * f + 4 * g);
            const float4 qv = __builtin_bit_cast(float4, qf[f]);
            s[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.x, qv.x, s[kb], 0, 0, 0);
            s[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.y, qv.y, s[kb], 0, 0, 0);
            s[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.z, qv.z, s[kb], 0, 0, 0);
            s[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.w, qv.w, s[kb], 0, 0, 0);
          }
        }
      }

      // ---- causal mask, online softmax (log2 domain, per query column)
      float p[4][4];
      float mt = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kt0 + 16 * kb + 4 * g + i;
          const float x = s[kb][i] * a.scale_log2;
          p[kb][i] = key <= qpos ? x : -INFINITY;
          mt = fmaxf(mt, p[kb][i]);
        }
      mt = cross_group_max(mt);
      const float m_new = fmaxf(m_run, mt);   // finite: key 0 is visible to every query
      const float alpha = fast_exp2(m_run - m_new);
      m_run = m_new;
      float ps = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[kb][i] = fast_exp2(p[kb][i] - m_new);
          ps += p[kb][i];
        }
      l_part = l_part * alpha + ps;
#pragma unroll
      for (int db = 0; db < NDB; ++db) oacc[db] *= alpha;

      // ---- O^T += V^T P^T
      if constexpr (kBF16) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          uint4 pb;
          pb.x = (uint32_t)f32_to_bf16(p[2 * c][0]) | ((uint32_t)f32_to_bf16(p[2 * c][1]) << 16);
          pb.y = (uint32_t)f32_to_bf16(p[2 * c][2]) | ((uint32_t)f32_to_bf16(p[2 * c][3]) << 16);
          pb.z = (uint32_t)f32_to_bf16(p[2 * c + 1][0]) | ((uint32_t)f32_to_bf16(p[2 * c + 1][1]) << 16);
          pb.w = (uint32_t)f32_to_bf16(p[2 * c + 1][2]) | ((uint32_t)f32_to_bf16(p[2 * c + 1][3]) << 16);
#pragma unroll
          for (int db = 0; db < NDB; ++db) {
            const T* vrow = &vt_lds[(16 * db + col) * VROW + 32 * c + 4 * g];
            const uint2 v0 = *reinterpret_cast<const uint2*>(vrow);
            const uint2 v1 = *reinterpret_cast<const uint2*>(vrow + 16);
            const uint4 va = make_uint4(v0.x, v0.y, v1.x, v1.y);
            oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, va),
                                                               __builtin_bit_cast(bf16x8_t, pb),
                                                               oacc[db], 0, 0, 0);
          }
        }
      } else {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int db = 0; db < NDB; ++db) {
            const float4 vv = *reinterpret_cast<const float4*>(
                &vt_lds[(16 * db + col) * VROW + 16 * kb + 4 * g]);
            oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.x, p[kb][0], oacc[db], 0, 0, 0);
            oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.y, p[kb][1], oacc[db], 0, 0, 0);
            oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.z, p[kb][2], oacc[db], 0, 0, 0);
            oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.w, p[kb][3], oacc[db], 0, 0, 0);
          }
      }
    }
    __syncthreads();
  }

  // ---- normalise and store: lane holds out[qi, h, 16*db + 4*g + 0..3]
  const float l = cross_group_sum(l_part);
  if (!q_ok) return;
  const float inv = 1.f / l;
  T* orow = reinterpret_cast<T*>(a.out) + (int64_t)qi * a.o_st + (int64_t)h * a.o_sh;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    const int d0 = 16 * db + 4 * g;
    if (d0 >= a.D) continue;
    if constexpr (kBF16) {
      uint2 w;
      w.x = (uint32_t)f32_to_bf16(oacc[db][0] * inv) | ((uint32_t)f32_to_bf16(oacc[db][1] * inv) << 16);
      w.y = (uint32_t)f32_to_bf16(oacc[db][2] * inv) | ((uint32_t)f32_to_bf16(oacc[db][3] * inv) << 16);
      *reinterpret_cast<uint2*>(orow + d0) = w;
    } else {
      *reinterpret_cast<float4*>(orow + d0) =
          make_float4(oacc[db][0] * inv, oacc[db][1] * inv, oacc[db][2] * inv, oacc[db][3] * inv);
    }
  }
}

template <typename T, int DP>
hipError_t launch_dp(const PrefillArgs& a, int waves, hipStream_t stream) {
  const int qb = 16 * waves;
  const dim3 grid((unsigned)((a.T + qb - 1) / qb), (unsigned)a.H);
  if (waves == 4)
    hipLaunchKernelGGL((paged_prefill_mfma<T, DP, 4>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((paged_prefill_mfma<T, DP, 2>), grid, dim3(128), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

int prefill_head_dim_bucket(int dtype_is_bf16, int D) {
  if (D <= 32) return 32;
  if (D <= 64) return 64;
  if (D <= 128) return 128;
  if (dtype_is_bf16 && D <= 256) return 256;
  return 0;
}

hipError_t launch_paged_prefill(const PrefillArgs& a, bool bf16, int dp, int waves,
                                hipStream_t stream) {
  if (bf16) {
    switch (dp) {
      case 32: return launch_dp<bf16_t, 32>(a, waves, stream);
      case 64: return launch_dp<bf16_t, 64>(a, waves, stream);
      case 128: return launch_dp<bf16_t, 128>(a, waves, stream);
      case 256: return launch_dp<bf16_t, 256>(a, waves, stream);
    }
  } else {
    switch (dp) {
      case 32: return launch_dp<float, 32>(a, waves, stream);
      case 64: return launch_dp<float, 64>(a, waves, stream);
      case 128: return launch_dp<float, 128>(a, waves, stream);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace mgi
