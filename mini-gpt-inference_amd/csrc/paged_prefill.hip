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
// Work split: one workgroup per (query tile, head); each wavefront owns a
// block of 16 query rows. Keys stream through LDS in tiles of 64 (K
// row-major, V transposed, two stages so one barrier per tile suffices).
// Each wave computes S^T = K Q^T and O^T += V^T P^T with 16x16 MFMA tiles,
// so a lane's accumulator column is one query row: the online-softmax state
// (max, sum) is per lane and P needs no transpose. With split keys (a short
// chunk after a long prefix), blockIdx.y selects a partition of the query
// tile's keys and rows spanning several partitions write fp32 partials that
// paged_decode_merge combines.
//
// Numerics: fp32 accumulation and softmax in the log2 domain; bf16 and f16
// inputs use v_mfma_f32_16x16x32_bf16 / _f16 with P rounded to the input
// type for the PV product, fp32 inputs use v_mfma_f32_16x16x4_f32 (full fp32
// products).
#include <cstdlib>

#include "mgi_common.h"
#include "mgi_internal.h"
#include "minivllm_hip.h"

namespace mgi {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTileKeys = 64;  // keys per LDS tile

template <typename T> struct PF;
// Row paddings (elements) of the K and V^T LDS tiles. 16-byte multiples keep
// every 16-byte access aligned; the values were chosen by measurement on
// MI355X (unpadded K rows cost 38%; 16/16 beat 8/8 by 8%) and keep two
// workgroups' double-buffered tiles within one CU's LDS.
template <> struct PF<bf16_t> {
  static constexpr int kChunk = 8;  // elements per 16-byte chunk
  static constexpr int kKPad = 16;
  static constexpr int kVPad = 16;
};
template <> struct PF<f16_t> : PF<bf16_t> {};
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

// The kernels take tile maxima over raw scores s (masked ones -inf) and
// scale them afterwards, which needs a positive scale c. softmax(c s) =
// softmax(|c| (-s)) for c < 0, and softmax(1 (0 s)) for c = 0. So the query
// fragments are negated for c < 0 (exactly, by flipping the sign bit of every
// T element of the 32-bit words) or zeroed for c = 0, and query_scale(c)
// replaces c.
template <typename T>
__device__ __forceinline__ uint4 query_sign(uint4 x, float c) {
  if (c == 0.f) return make_uint4(0, 0, 0, 0);
  const uint32_t m = c < 0.f ? (sizeof(T) == 2 ? 0x80008000u : 0x80000000u) : 0u;
  return make_uint4(x.x ^ m, x.y ^ m, x.z ^ m, x.w ^ m);
}
__device__ __forceinline__ float query_scale(float c) { return c == 0.f ? 1.f : fabsf(c); }

// Element offsets of key `key`'s K and V rows (relative to the head's base
// in the layer), or -1 for keys past the chunk or invalid table entries.
struct KeyRows {
  int64_t k, v;
};
__device__ __forceinline__ KeyRows key_rows(const PrefillArgs& a, int key, int kv_end) {
  if (key >= kv_end) return KeyRows{-1, -1};
  int blk, off;
  if (a.s_shift >= 0) {
    blk = key >> a.s_shift;
    off = key & (a.S - 1);
  } else {
    blk = key / a.S;
    off = key - blk * a.S;
  }
  const int64_t phys = load_index(a.bt, a.bt_i64, (int64_t)blk * a.bt_s);
  if (phys < 0 || phys >= a.N) return KeyRows{-1, -1};
  return KeyRows{phys * a.k_sn + off * a.k_ss, phys * a.v_sn + off * a.v_ss};
}

// Online-softmax reference maxima move only when a tile's maximum exceeds
// them by more than this (log2 units), so exponentials stay <= 2^8 and the
// accumulators are rescaled on few tiles.
constexpr float kRescaleSlack = 8.f;

// The 2-byte input types: a 16x16x32 MFMA on eight packed values per lane and
// operand, and a two-value pack with the hardware conversion (round to
// nearest even).
template <typename T> struct Mma16;
template <> struct Mma16<bf16_t> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  __device__ static __forceinline__ f32x4_t mfma(uint4 a, uint4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c,
                                                   0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    const v2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
};
template <> struct Mma16<f16_t> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  __device__ static __forceinline__ f32x4_t mfma(uint4 a, uint4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a), __builtin_bit_cast(v8, b), c,
                                                  0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    const v2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
};
template <> struct Mma16<float> {  // never called: fp32 takes the 16x16x4 path
  __device__ static __forceinline__ f32x4_t mfma(uint4, uint4, f32x4_t c) { return c; }
  __device__ static __forceinline__ uint32_t pack2(float, float) { return 0u; }
};

// Column of key k (0..63) in a 2-byte V^T tile row. Keys 32c + 16h + 4g + i
// sit at 32c + 8g + 4h + i, so the eight keys one lane feeds to a PV MFMA
// (4g+i and 16+4g+i of a 32-key slice) are one 16-byte LDS read.
__device__ __forceinline__ int vt_col_bf16(int k) {
  return (k & 32) | ((k & 12) << 1) | ((k & 16) >> 2) | (k & 3);
}

// T: element type; DP: head dim padded to the MFMA K width (D <= DP);
// WAVES: wavefronts per workgroup; QPW: 16-row query blocks per wavefront.
template <typename T, int DP, int WAVES, int QPW>
__global__ __launch_bounds__(64 * WAVES) void paged_prefill_mfma(const PrefillArgs a) {
  using E = PF<T>;
  constexpr int CH = E::kChunk;
  constexpr int CPR = DP / CH;                 // 16-byte chunks per key row
  constexpr int KROW = DP + E::kKPad;          // K tile row stride (elements)
  constexpr int VROW = kTileKeys + E::kVPad;   // V^T tile row stride (elements)
  constexpr int NT = 64 * WAVES;
  constexpr int ITEMS = 16 * CPR;              // (4-key group, chunk) pairs per tile
  constexpr int IPT = (ITEMS + NT - 1) / NT;
  constexpr int QB = 16 * QPW * WAVES;         // query rows per workgroup
  constexpr bool k16 = sizeof(T) == 2;             // bf16 or f16
  using MM = Mma16<T>;
  constexpr int NQF = k16 ? DP / 32 : DP / 16;     // Q fragments (16 bytes each)
  constexpr int NDB = DP / 16;                     // 16-wide head-dim blocks of O^T

  // Two stages: tile t is read from one while tile t+1 is written to the other.
  __shared__ __align__(16) T k_lds[2][kTileKeys * KROW];
  __shared__ __align__(16) T vt_lds[2][DP * VROW];
  __shared__ KeyRows slots[2][kTileKeys];  // tile t's rows in stage t & 1
  __shared__ uint64_t slot_valid[4];      // tile t in stage t & 3; bit k: key k has K and V rows

  // 1-D grid of nq * H workgroups, dispatched round-robin over the XCDs
  // (workgroup id mod 8). With H a multiple of 8, every query tile of head h
  // runs on XCD h mod 8, so each XCD's L2 holds the K/V of H/8 heads only.
  // Within a head, the longest (latest) query tiles go first. When the whole
  // grid is resident at once (two workgroups per CU, pair_round = CUs per
  // XCD), the second round of an XCD's workgroups runs in the opposite
  // order, so the two workgroups that share a CU have query tiles qt and
  // nq-1-qt and about the same causal work together.
  const int nq = (a.T + QB - 1) / QB;
  const int wg = (int)blockIdx.x;
  int h, qr;
  if ((a.H & 7) == 0) {
    int j = wg >> 3;
    if (a.pair_round > 0 && (j / a.pair_round) & 1) {
      const int lo = j - j % a.pair_round;
      const int hi = min(lo + a.pair_round, (a.H >> 3) * nq);
      j = hi - 1 - (j - lo);
    }
    h = (wg & 7) + 8 * (j / nq);
    qr = j % nq;
  } else {
    h = wg / nq;
    qr = wg % nq;
  }
  const int qt = nq - 1 - qr;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 15, g = lane >> 4;
  const int qw0 = qt * QB + wave * 16 * QPW;
  const int kv_end = a.start + min(a.T, (qt + 1) * QB);
  // Key partition (blockIdx.y) when the keys are split: this workgroup takes
  // key tiles [tb, te) of its query tile's range and writes partials for the
  // rows whose keys span several partitions.
  const int part = (int)blockIdx.y;
  const int ntiles_all = (kv_end + kTileKeys - 1) / kTileKeys;
  const int tpp = a.part_keys > 0 ? a.part_keys / kTileKeys : ntiles_all;
  const int tb = part * tpp;
  if (tb >= ntiles_all) return;  // uniform: this query tile needs fewer partitions
  const int key0 = tb * kTileKeys;
  const bool wave_active = qw0 < a.T;
  const int wave_first = a.start + qw0;
  const int wave_last = a.start + min(a.T, qw0 + 16 * QPW) - 1;
  const int ntiles = min(ntiles_all, tb + tpp) - tb;  // this workgroup's tiles

  int qi[QPW], qpos[QPW];
#pragma unroll
  for (int b = 0; b < QPW; ++b) {
    qi[b] = qw0 + 16 * b + col;
    qpos[b] = a.start + (qi[b] < a.T ? qi[b] : a.T - 1);
  }

  // ---- this lane's query fragments (zero past the chunk or past D)
  uint4 qf[QPW][NQF];
#pragma unroll
  for (int b = 0; b < QPW; ++b) {
    const bool ok = qi[b] < a.T;
    const T* qrow = reinterpret_cast<const T*>(a.q) + (int64_t)(ok ? qi[b] : 0) * a.q_st +
                    (int64_t)h * a.q_sh;
#pragma unroll
    for (int f = 0; f < NQF; ++f) {
      const int d = k16 ? 32 * f + 8 * g : 16 * f + 4 * g;
      qf[b][f] = (ok && d < a.D) ? *reinterpret_cast<const uint4*>(qrow + d) : make_uint4(0, 0, 0, 0);
      qf[b][f] = query_sign<T>(qf[b][f], a.scale_log2);
    }
  }

  const T* kb_ = reinterpret_cast<const T*>(a.k) + (int64_t)h * a.k_sh;
  const T* vb_ = reinterpret_cast<const T*>(a.v) + (int64_t)h * a.v_sh;

  // Staging registers: item j of this thread covers 4 keys x one chunk, for K
  // (keys vary slowest: lanes sweep the head dim) and V (lanes sweep keys).
  // Two sets: tile t is staged in set t & 1, loaded two tiles ahead.
  uint4 kr0[IPT][4], vr0[IPT][4], kr1[IPT][4], vr1[IPT][4];
  auto load_tile = [&](uint4 (&kr)[IPT][4], uint4 (&vr)[IPT][4], int sb) {
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      const int it = tid + NT * j;
      const bool in = (ITEMS % NT == 0) || it < ITEMS;
      const int kq_k = it / CPR, dc_k = it % CPR;
      const int kq_v = it % 16, dc_v = it / 16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t ko = slots[sb][4 * kq_k + r].k;
        const int64_t vo = slots[sb][4 * kq_v + r].v;
        const bool okk = in && ko >= 0 && dc_k * CH < a.D;
        const bool okv = in && vo >= 0 && dc_v * CH < a.D;
        kr[j][r] = okk ? *reinterpret_cast<const uint4*>(kb_ + ko + dc_k * CH) : make_uint4(0, 0, 0, 0);
        vr[j][r] = okv ? *reinterpret_cast<const uint4*>(vb_ + vo + dc_v * CH) : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto store_tile = [&](const uint4 (&kr)[IPT][4], const uint4 (&vr)[IPT][4], int buf) {
    T* kl = k_lds[buf];
    T* vl = vt_lds[buf];
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      const int it = tid + NT * j;
      if (!((ITEMS % NT == 0) || it < ITEMS)) continue;
      const int kq_k = it / CPR, dc_k = it % CPR;
      const int kq_v = it % 16, dc_v = it / 16;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<uint4*>(&kl[(4 * kq_k + r) * KROW + dc_k * CH]) = kr[j][r];
      if constexpr (k16) {
        // 8 head dims x 4 keys -> eight 4-key runs of V^T rows. Each packed
        // pair takes the same 16-bit half of one word of two keys' rows
        // (v_perm_b32 byte select: 0-3 from the second operand, 4-7 from the first).
        const int vc = vt_col_bf16(4 * kq_v);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          auto word = [&](const uint4& x) {
            const int w = e >> 1;
            return w == 0 ? x.x : w == 1 ? x.y : w == 2 ? x.z : x.w;
          };
          const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
          uint2 pk;
          pk.x = __builtin_amdgcn_perm(word(vr[j][1]), word(vr[j][0]), sel);
          pk.y = __builtin_amdgcn_perm(word(vr[j][3]), word(vr[j][2]), sel);
          *reinterpret_cast<uint2*>(&vl[(8 * dc_v + e) * VROW + vc]) = pk;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          auto word = [&](const uint4& x) { return e == 0 ? x.x : e == 1 ? x.y : e == 2 ? x.z : x.w; };
          uint4 pk = make_uint4(word(vr[j][0]), word(vr[j][1]), word(vr[j][2]), word(vr[j][3]));
          *reinterpret_cast<uint4*>(&vl[(4 * dc_v + e) * VROW + 4 * kq_v]) = pk;
        }
      }
    }
  };

  f32x4_t oacc[QPW][NDB];
  float m_run[QPW], l_part[QPW];
#pragma unroll
  for (int b = 0; b < QPW; ++b) {
#pragma unroll
    for (int i = 0; i < NDB; ++i) oacc[b][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    m_run[b] = -INFINITY;
    l_part[b] = 0.f;
  }

  auto compute = [&](int buf, int vb, int kt0) {
    const T* kl = k_lds[buf];
    const T* vl = vt_lds[buf];
    // ---- S^T blocks: lane holds keys kt0 + 16*kb + 4*g + i of query column `col`
    f32x4_t s[QPW][4];
#pragma unroll
    for (int b = 0; b < QPW; ++b)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) s[b][kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const T* krow = &kl[(16 * kb + col) * KROW];
#pragma unroll
      for (int f = 0; f < NQF; ++f) {
        if constexpr (k16) {
          const uint4 kv = *reinterpret_cast<const uint4*>(krow + 32 * f + 8 * g);
#pragma unroll
          for (int b = 0; b < QPW; ++b) s[b][kb] = MM::mfma(kv, qf[b][f], s[b][kb]);
        } else {
          const float4 kv = *reinterpret_cast<const float4*>(krow + 16 * f + 4 * g);
#pragma unroll
          for (int b = 0; b < QPW; ++b) {
            const float4 qv = __builtin_bit_cast(float4, qf[b][f]);
            s[b][kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.x, qv.x, s[b][kb], 0, 0, 0);
            s[b][kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.y, qv.y, s[b][kb], 0, 0, 0);
            s[b][kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.z, qv.z, s[b][kb], 0, 0, 0);
            s[b][kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.w, qv.w, s[b][kb], 0, 0, 0);
          }
        }
      }
    }

    // ---- causal mask (diagonal tiles) and invalid-key mask, online softmax
    // per query column. Raw scores s; the log2-domain score is
    // s * query_scale(scale_log2) (the query carries the scale's sign, so the
    // maximum of raw scores gives the maximum of scaled ones).
    // The tile's validity mask is wave-uniform: read it into scalar registers
    // so interior tiles take a branch with no masking work at all.
    const uint64_t vm_lds = slot_valid[vb];
    const uint32_t vm_lo = __builtin_amdgcn_readfirstlane((uint32_t)vm_lds);
    const uint32_t vm_hi = __builtin_amdgcn_readfirstlane((uint32_t)(vm_lds >> 32));
    const bool full = kt0 + kTileKeys - 1 <= wave_first && (vm_lo & vm_hi) == 0xffffffffu;
    const float c = query_scale(a.scale_log2);
    float p[QPW][4][4];
    if (full) {
#pragma unroll
      for (int b = 0; b < QPW; ++b)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) p[b][kb][i] = s[b][kb][i];
    } else {
      // This lane's keys are 16*kb + 4*g + i: gather their validity bits once.
      const uint64_t vm = ((uint64_t)vm_hi << 32) | vm_lo;
      uint32_t lv = 0;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) lv |= ((uint32_t)(vm >> (16 * kb + 4 * g)) & 0xfu) << (4 * kb);
#pragma unroll
      for (int b = 0; b < QPW; ++b)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bool vis = kt0 + 16 * kb + 4 * g + i <= qpos[b] && ((lv >> (4 * kb + i)) & 1u);
            p[b][kb][i] = vis ? s[b][kb][i] : -INFINITY;
          }
    }
#pragma unroll
    for (int b = 0; b < QPW; ++b) {
      float mt = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) mt = fmaxf(mt, p[b][kb][i]);
      // The reference maximum (uniform over the four lanes of a column) moves,
      // and the state is rescaled, only when some lane's tile maximum outgrows
      // it by more than the slack; only then is the column maximum reduced
      // across lanes. A column with nothing visible yet keeps m = -inf and a
      // zero state.
      mt *= c;
      if (__builtin_amdgcn_ballot_w64(mt > m_run[b] + kRescaleSlack) != 0) {
        mt = cross_group_max(mt);
        const float m_new = fmaxf(m_run[b], mt);
        const float alpha = m_run[b] == -INFINITY ? 0.f : fast_exp2(m_run[b] - m_new);
        m_run[b] = m_new;
        l_part[b] *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db) oacc[b][db] *= alpha;
      }
      const float neg_m = m_run[b] == -INFINITY ? 0.f : -m_run[b];
      float ps = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[b][kb][i] = fast_exp2(fmaf(p[b][kb][i], c, neg_m));
          ps += p[b][kb][i];
        }
      l_part[b] += ps;
    }

    // ---- O^T += V^T P^T
    if constexpr (k16) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        uint4 pb[QPW];
#pragma unroll
        for (int b = 0; b < QPW; ++b)
          pb[b] = make_uint4(MM::pack2(p[b][2 * c][0], p[b][2 * c][1]),
                             MM::pack2(p[b][2 * c][2], p[b][2 * c][3]),
                             MM::pack2(p[b][2 * c + 1][0], p[b][2 * c + 1][1]),
                             MM::pack2(p[b][2 * c + 1][2], p[b][2 * c + 1][3]));
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const uint4 va = *reinterpret_cast<const uint4*>(&vl[(16 * db + col) * VROW + 32 * c + 8 * g]);
#pragma unroll
          for (int b = 0; b < QPW; ++b) oacc[b][db] = MM::mfma(va, pb[b], oacc[b][db]);
        }
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const float4 vv = *reinterpret_cast<const float4*>(&vl[(16 * db + col) * VROW + 16 * kb + 4 * g]);
#pragma unroll
          for (int b = 0; b < QPW; ++b) {
            oacc[b][db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.x, p[b][kb][0], oacc[b][db], 0, 0, 0);
            oacc[b][db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.y, p[b][kb][1], oacc[b][db], 0, 0, 0);
            oacc[b][db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.z, p[b][kb][2], oacc[b][db], 0, 0, 0);
            oacc[b][db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.w, p[b][kb][3], oacc[b][db], 0, 0, 0);
          }
        }
    }
  };

  // Wave 0 (tid < 64, all lanes active) publishes a tile's K/V row offsets
  // and which of its keys have them.
  auto put_slots = [&](int tile, const KeyRows& rows) {
    slots[tile & 1][tid] = rows;
    const uint64_t vm = __builtin_amdgcn_ballot_w64(rows.k >= 0 && rows.v >= 0);
    if (tid == 0) slot_valid[tile & 3] = vm;
  };
  KeyRows slot_next{-1, -1};
  if constexpr (k16) {
    // ---- pipeline (2-byte types): tile t+1 waits in registers while tile t
    // is computed, and the loads of tile t+2 are in flight (two compute steps
    // from load to use); block-table rows are resolved one tile before their
    // loads. Measured on MI355X: 16% faster than one tile ahead for a 512-row
    // chunk after a 512-token prefix, equal on 2048-row chunks.
    if (tid < kTileKeys) {
      put_slots(0, key_rows(a, key0 + tid, kv_end));
      put_slots(1, key_rows(a, key0 + kTileKeys + tid, kv_end));
      slot_next = key_rows(a, key0 + 2 * kTileKeys + tid, kv_end);
    }
    __syncthreads();
    load_tile(kr0, vr0, 0);
    if (ntiles > 1) load_tile(kr1, vr1, 1);
    store_tile(kr0, vr0, 0);
    __syncthreads();  // every wave has read tile 0's rows (stage 0)
    if (tid < kTileKeys) {
      put_slots(2, slot_next);
      slot_next = key_rows(a, key0 + 3 * kTileKeys + tid, kv_end);
    }
    __syncthreads();
    if (ntiles > 2) load_tile(kr0, vr0, 0);  // tile 2 (rows stage 2 & 1 = 0)

    // One step: compute tile t, stage tile t+1 (held in set kn/vn) into LDS,
    // publish the rows of tile t+3, then load tile t+3 into the freed set.
    auto step = [&](int t, uint4 (&kn)[IPT][4], uint4 (&vn)[IPT][4]) {
      const int kt0 = key0 + t * kTileKeys;
      if (wave_active && kt0 <= wave_last) compute(t & 1, t & 3, kt0);
      if (t + 1 < ntiles) store_tile(kn, vn, (t + 1) & 1);
      if (tid < kTileKeys && t + 3 < ntiles) {
        put_slots(t + 3, slot_next);
        slot_next = key_rows(a, key0 + (t + 4) * kTileKeys + tid, kv_end);
      }
      __syncthreads();
      if (t + 3 < ntiles) load_tile(kn, vn, (t + 3) & 1);
    };
    for (int t = 0; t < ntiles; t += 2) {
      step(t, kr1, vr1);
      if (t + 1 < ntiles) step(t + 1, kr0, vr0);
    }
  } else {
    // ---- pipeline (fp32, whose registers allow one staging set): tile t+1 is
    // in registers while tile t is computed; its block-table rows are in LDS
    // two tiles ahead.
    if (tid < kTileKeys) {
      put_slots(0, key_rows(a, key0 + tid, kv_end));
      if (ntiles > 1) slot_next = key_rows(a, key0 + kTileKeys + tid, kv_end);
    }
    __syncthreads();
    load_tile(kr0, vr0, 0);
    if (tid < kTileKeys) {
      put_slots(1, slot_next);
      if (ntiles > 2) slot_next = key_rows(a, key0 + 2 * kTileKeys + tid, kv_end);
    }
    store_tile(kr0, vr0, 0);
    __syncthreads();
    if (ntiles > 1) load_tile(kr0, vr0, 1);

    for (int t = 0; t < ntiles; ++t) {
      const int kt0 = key0 + t * kTileKeys;
      if (wave_active && kt0 <= wave_last) compute(t & 1, t & 3, kt0);
      if (t + 1 < ntiles) {
        if (tid < kTileKeys) {
          put_slots(t + 2, slot_next);
          if (t + 3 < ntiles) slot_next = key_rows(a, key0 + (t + 3) * kTileKeys + tid, kv_end);
        }
        store_tile(kr0, vr0, (t + 1) & 1);
      }
      __syncthreads();
      if (t + 2 < ntiles) load_tile(kr0, vr0, t & 1);
    }
  }

  // ---- normalise and store: lane holds out[qi, h, 16*db + 4*g + 0..3]. With
  // split keys, a row whose keys span several partitions writes its
  // unnormalised state (max, sum, O) to slot (qi * H + h) * max_parts + part,
  // the layout paged_decode_merge combines (a row at context start + qi + 1,
  // partitions of part_keys keys); a row inside one partition is stored here.
#pragma unroll
  for (int b = 0; b < QPW; ++b) {
    const float l = cross_group_sum(l_part[b]);
    if (qi[b] >= a.T) continue;
    if (a.part_keys > 0) {
      const int np = (a.start + qi[b] + a.part_keys) / a.part_keys;  // ceil((start + qi + 1) / part_keys)
      if (part >= np) continue;  // the row's keys end before this partition
      if (np > 1) {
        const size_t slot = ((size_t)qi[b] * a.H + h) * a.max_parts + part;
        if (g == 0) a.ws_ml[slot] = make_float2(m_run[b], l);
        float* wa = a.ws_acc + slot * a.D;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const int d0 = 16 * db + 4 * g;
          if (d0 >= a.D) continue;
          *reinterpret_cast<float4*>(wa + d0) =
              make_float4(oacc[b][db][0], oacc[b][db][1], oacc[b][db][2], oacc[b][db][3]);
        }
        continue;
      }
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;  // no visible valid key: zeros
    T* orow = reinterpret_cast<T*>(a.out) + (int64_t)qi[b] * a.o_st + (int64_t)h * a.o_sh;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int d0 = 16 * db + 4 * g;
      if (d0 >= a.D) continue;
      if constexpr (k16) {
        uint2 w;
        w.x = MM::pack2(oacc[b][db][0] * inv, oacc[b][db][1] * inv);
        w.y = MM::pack2(oacc[b][db][2] * inv, oacc[b][db][3] * inv);
        *reinterpret_cast<uint2*>(orow + d0) = w;
      } else {
        *reinterpret_cast<float4*>(orow + d0) = make_float4(oacc[b][db][0] * inv, oacc[b][db][1] * inv,
                                                            oacc[b][db][2] * inv, oacc[b][db][3] * inv);
      }
    }
  }
}

// ------------------------------------------------------------------------
// Direct-to-LDS variant (2-byte types, head dims 64 and 128, power-of-two
// block sizes of at least 16). Same grid mapping, softmax and outputs as
// paged_prefill_mfma; what changes is how key tiles reach the matrix cores
// and how little per-tile VALU work the wavefronts spend (VALU issue, not
// the matrix cores, bounds this kernel):
//   * The softmax denominators come out of the PV products (a block of ones
//     beside V^T), as sums of the 2-byte P the outputs accumulate, and a
//     tile's rescale check is one compare of its raw maximum per 16-row
//     block against a threshold kept with the state.
//   * A key tile is 64 keys = four 16-key granules, and a granule lies in one
//     pool block (S is a power of two >= 16). The workgroup keeps a window of
//     the block table in LDS as one int per granule: G = block * (S / 16) +
//     (offset in block) / 16, or -1 where the table entry is invalid or the
//     granule starts past the chunk. One LDS read per step gives lanes
//     0 .. 4 GROUPS - 1 the step's granules; what follows from them is
//     wave-uniform scalar work.
//   * K and V tiles are copied from HBM straight into LDS by 16-byte
//     global_load_lds copies (one instruction moves 1 KiB: RPG whole key
//     rows); each copying wavefront takes a contiguous run of a tile's rows.
//     When a tile's granules are all valid and inside the chunk, a copy is
//     the granule's base address in scalar registers plus a per-lane 32-bit
//     offset fixed for the whole loop. Otherwise each lane picks its source
//     row, and keys past the chunk, invalid granules and head dims past D
//     read a zero row.
//   * Rows store their 16-byte chunk c at c ^ ks(r) (K) and c ^ vs(r) (V),
//     swizzles chosen by measuring these kernels' read sequences on MI355X:
//     ks(r) = (r & 3) | ((r >> 1) & (CPR - 4)); vs(r) = 2 (r & 3) |
//     8 ((r >> 3) & 1) for 16-chunk rows, 2 (r & 3) for 8-chunk rows.
//   * S^T = K Q^T reads the A operand (16 keys x 8 head dims per lane) as one
//     16-byte row read; the A rows of key block kb = 2c + h are the keys
//     32c + 8(r/4) + 4h + r%4, so the S^T column a lane holds for blocks 2c
//     and 2c+1 is exactly the 8 keys 32c + 8g .. 32c + 8g + 7 that the PV
//     product takes as its B operand (P^T), packed in register order.
//   * O^T += V^T P^T reads its A operand (V^T: 16 head dims x those 8 keys)
//     with two ds_read_b64_tr_b16: in each 16-lane group, lane i receives
//     element i % 4 of the 4-element chunks addressed by lanes 4j + i/4,
//     j = 0..3 (the instruction's lane layout, measured on MI355X), so lanes
//     addressing V rows (keys) 8g + 4u + j at head dims 16db + 4q give lane i
//     head dim 16db + i of four consecutive keys.
//   * STAGES tiles in flight (per group), one barrier per step. The loop body
//     exists once per stage, so the LDS offsets of the operand reads are
//     immediates. The copies are inline assembly, so the compiler adds no
//     waits of its own for them; the loop waits for them explicitly (each
//     wave's copies, then the barrier).
template <int CPR>
__device__ __forceinline__ int k_swz(int row) {
  return (row & 3) | ((row >> 1) & (CPR - 4));
}
template <int CPR>
__device__ __forceinline__ int v_swz(int row) {
  return CPR == 16 ? (2 * (row & 3)) | (8 * ((row >> 3) & 1)) : 2 * (row & 3);
}

// Source of the zero rows the copies read for keys that must contribute nothing.
__device__ __align__(16) const unsigned char kZeroRow[512] = {0};

template <typename T> struct TrRead;
template <> struct TrRead<bf16_t> {
  typedef __bf16 v4 __attribute__((ext_vector_type(4)));
  // From an LDS byte address: constant terms added to it fold into the
  // instruction's offset field.
  __device__ static __forceinline__ uint2 at(uint32_t addr) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                                         (__attribute__((address_space(3))) v4*)(uintptr_t)addr));
  }
};
template <> struct TrRead<f16_t> {
  typedef __fp16 v4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
  __device__ static __forceinline__ uint2 at(uint32_t addr) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                                         (__attribute__((address_space(3))) v4*)(uintptr_t)addr));
  }
};

// One 16-byte copy per lane from global memory into LDS at lds_base + 16 *
// lane (lds_base wave-uniform): global_load_lds_dwordx4 from a per-lane
// address, or from a wave-uniform base plus a per-lane 32-bit offset. The
// instruction takes its LDS base from M0; the "{m0}" operand has the compiler
// set M0 to lds_base before the statement (the asm only reads it), and the
// s_nop is the wait state an LDS copy needs after an SALU write of M0. The
// copy stays opaque to the compiler's wait-count tracking: the pipeline below
// counts its copies itself (wait_and_barrier). With the compiler's own
// __builtin_amdgcn_global_load_lds the kernel measured 4% slower on MI355X
// (2048 rows after 2048: 70.5-71.1 against 67.8-68.0 us on one box), as the
// compiler then drains every LDS read (lgkmcnt(0)) before MFMAs that use
// them.
__device__ __forceinline__ void copy16_to_lds(const void* src, uint32_t lds_base) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds_base) : "memory");
}
__device__ __forceinline__ void copy16_to_lds(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_base)
               : "memory");
}

// Waits until at most N of this wave's vector-memory instructions are
// outstanding and all its LDS and scalar memory instructions are done, then
// joins the workgroup barrier.
template <int N>
__device__ __forceinline__ void wait_and_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));  // vmcnt(N) expcnt(7) lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)(p);
}

constexpr int kGranuleWindow = 1024;  // 16-key granules of the block table a workgroup keeps in LDS

template <int V> struct Stage {
  static constexpr int value = V;
};

// Calls f(Stage<I>{}) for I = B .. E - 1.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(Stage<B>{});
    static_for<B + 1, E>(f);
  }
}

// GROUPS = 2 splits the workgroup's wavefronts into two groups of WAVES that
// cover the same query rows: group r computes the key tiles t with
// t % 2 == r, each through its own STAGES tile buffers, and at the end group
// 1 hands its softmax state (running max, partial sums, unnormalised output)
// to group 0 through LDS, which merges and stores. Group 0's wavefronts issue
// the copies of both groups' tiles. A wavefront can then own 32 query rows
// (each K and V read from LDS feeds two products) while two wavefronts share
// every SIMD.
//
// PAIRED (QPW = 2) balances the causal triangle: the chunk's rows are cut
// into half tiles of 16 WAVES rows, and the workgroup for pair p takes half
// tiles p and nh - 1 - p (nh half tiles), a wavefront's block 0 in the first
// and block 1 in the second. Every pair then holds about the same number of
// (row block, key tile) products, where plain 2-block tiles range from the
// chunk's shortest chain to its longest and the longest sets the kernel's
// time. Key tiles past block 0's last row run block 1 alone.
template <typename T, int DP, int WAVES, int QPW, int STAGES, int GROUPS, bool PAIRED = false>
__global__ __launch_bounds__(64 * WAVES * GROUPS) void paged_prefill_tr(const PrefillArgs a) {
  static_assert(sizeof(T) == 2 && (DP == 64 || DP == 128), "2-byte types, head dim 64 or 128");
  static_assert(WAVES == 2 || WAVES == 4 || WAVES == 8, "two, four or eight wavefronts per group");
  static_assert(STAGES >= 2 && STAGES <= 4, "two to four tiles in flight");
  static_assert(GROUPS == 1 || GROUPS == 2, "one or two groups");
  static_assert(!PAIRED || QPW == 2, "paired rows take two 16-row blocks per wavefront");
  constexpr int ROWB = DP * 2;               // bytes per key row
  constexpr int CPR = DP / 8;                // 16-byte chunks per key row
  constexpr int TILEB = kTileKeys * ROWB;    // bytes per K (or V) tile
  constexpr int RPG = 1024 / ROWB;           // key rows per copy
  constexpr int GPW = TILEB / 1024 / WAVES;  // copies per wave and tile (K or V)
  static_assert(GPW >= 1 && GPW * WAVES * 1024 == TILEB, "copies split evenly over the wavefronts");
  constexpr int RW = GPW * RPG;              // tile rows per wave
  constexpr int GRW = RW >= 16 ? RW / 16 : 1;  // granules a wave's rows lie in
  constexpr int CPGW = GPW / GRW;            // copies per such granule
  static_assert(2 * GPW * GROUPS * (STAGES - 2) < 64, "copies in flight fit the vmcnt immediate");
  constexpr int NT = 64 * WAVES * GROUPS;
  constexpr int QB = 16 * QPW * WAVES;       // query rows per workgroup
  constexpr int NQF = DP / 32;               // Q fragments (16 bytes each)
  constexpr int NDB = DP / 16;               // 16-wide head-dim blocks of O^T
  // LDS tile buffers: STAGES of K and of V per group.
  constexpr int KBUFS = GROUPS * STAGES;
  constexpr int VBUFS = GROUPS * STAGES;
  using MM = Mma16<T>;

  __shared__ __align__(1024) unsigned char k_lds[KBUFS * TILEB];
  __shared__ __align__(1024) unsigned char v_lds[VBUFS * TILEB];
  __shared__ __align__(16) int gran[kGranuleWindow];

  // Grid mapping: as paged_prefill_mfma (PAIRED: one workgroup per pair of
  // half tiles and head).
  constexpr int HB = 16 * WAVES;  // PAIRED: rows per half tile
  const int nh = (a.T + HB - 1) / HB;
  const int nq = PAIRED ? (nh + 1) / 2 : (a.T + QB - 1) / QB;
  const int wg = (int)blockIdx.x;
  int h, qr;
  if ((a.H & 7) == 0) {
    int j = wg >> 3;
    if (a.pair_round > 0 && (j / a.pair_round) & 1) {
      const int lo = j - j % a.pair_round;
      const int hi = min(lo + a.pair_round, (a.H >> 3) * nq);
      j = hi - 1 - (j - lo);
    }
    h = (wg & 7) + 8 * (j / nq);
    qr = j % nq;
  } else {
    h = wg / nq;
    qr = wg % nq;
  }
  const int qt = nq - 1 - qr;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wall = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = GROUPS == 1 ? 0 : wall / WAVES;  // group of this wavefront
  const int wave = GROUPS == 1 ? wall : wall % WAVES;  // wavefront within its group
  const int col = lane & 15, g = lane >> 4;
  // First chunk row of each of this wavefront's 16-row blocks (>= a.T: the
  // block has no rows) and the chunk rows this workgroup's keys reach.
  int rb[QPW], kv_rows;
  if constexpr (PAIRED) {
    const int hs = qt, hl = nh - 1 - qt;  // the middle half tile of an odd nh runs as block 1 alone
    rb[0] = hs < hl ? hs * HB + wave * 16 : a.T;
    rb[1] = hl * HB + wave * 16;
    kv_rows = (hl + 1) * HB;
  } else {
#pragma unroll
    for (int b = 0; b < QPW; ++b) rb[b] = qt * QB + wave * 16 * QPW + 16 * b;
    kv_rows = (qt + 1) * QB;
  }
  const int kv_end = a.start + min(a.T, kv_rows);
  const int part = (int)blockIdx.y;
  const int ntiles_all = (kv_end + kTileKeys - 1) / kTileKeys;
  const int tpp = a.part_keys > 0 ? a.part_keys / kTileKeys : ntiles_all;
  const int tb = part * tpp;
  if (tb >= ntiles_all) return;  // uniform: this query tile needs fewer partitions
  const int key0 = tb * kTileKeys;
  // Absolute positions of each block's first and last rows; the wavefront's
  // last position over the blocks that have rows (-1: none).
  int blk_first[QPW], blk_last[QPW];
  int wave_last = -1;
#pragma unroll
  for (int b = 0; b < QPW; ++b) {
    blk_first[b] = a.start + rb[b];
    blk_last[b] = a.start + min(a.T, rb[b] + 16) - 1;
    if (rb[b] < a.T) wave_last = max(wave_last, blk_last[b]);
  }
  const bool wave_active = wave_last >= 0;
  const int wave_first = blk_first[0];
  const int ntiles = min(ntiles_all, tb + tpp) - tb;
  const int nsteps = (ntiles + GROUPS - 1) / GROUPS;  // loop steps (every group takes them all)
  const int ntg = (ntiles - grp + GROUPS - 1) / GROUPS;  // tiles of this wave's group
  int qi[QPW], qpos[QPW];
#pragma unroll
  for (int b = 0; b < QPW; ++b) {
    qi[b] = rb[b] + col;
    qpos[b] = a.start + (qi[b] < a.T ? qi[b] : a.T - 1);
  }

  // ---- this lane's query fragments (zero past the chunk or past D)
  uint4 qf[QPW][NQF];
#pragma unroll
  for (int b = 0; b < QPW; ++b) {
    const bool ok = qi[b] < a.T;
    const T* qrow = reinterpret_cast<const T*>(a.q) + (int64_t)(ok ? qi[b] : 0) * a.q_st + (int64_t)h * a.q_sh;
#pragma unroll
    for (int f = 0; f < NQF; ++f) {
      const int d = 32 * f + 8 * g;
      qf[b][f] = (ok && d < a.D) ? *reinterpret_cast<const uint4*>(qrow + d) : make_uint4(0, 0, 0, 0);
      qf[b][f] = query_sign<T>(qf[b][f], a.scale_log2);
    }
  }

  // ---- granule window: granules gwin0 .. gwin0 + kGranuleWindow - 1 (gwin0 a
  // multiple of 4, as every tile's first granule is)
  const int gshift = a.s_shift - 4;
  const int gmask = (1 << gshift) - 1;
  const int sm = a.S - 1;
  int gwin0 = key0 >> 4;
  auto fill_window = [&]() {
    for (int i = tid; i < kGranuleWindow; i += NT) {
      const int key = (gwin0 + i) << 4;
      int v = -1;
      if (key < kv_end) {
        const int64_t e = load_index(a.bt, a.bt_i64, (int64_t)(key >> a.s_shift) * a.bt_s);
        if (e >= 0 && e < a.N) v = ((int)e << gshift) + ((key & sm) >> 4);
      }
      gran[i] = v;
    }
  };
  fill_window();
  __syncthreads();
  // The granules of this group's tile at step u (tile u * GROUPS + grp): lane
  // j of every four holds granule j. Moves the window first when step u's
  // tiles leave it, which drains the copies in flight; the condition depends
  // on u only, so the whole workgroup takes it together.
  auto tile_granules = [&](int u) -> int {
    const int s0 = (key0 >> 4) + 4 * GROUPS * u;  // first granule of the step's first tile
    if (s0 + 4 * GROUPS > gwin0 + kGranuleWindow) {
      __syncthreads();
      gwin0 = s0;
      fill_window();
      __syncthreads();
    }
    return gran[s0 - gwin0 + (lane & (4 * GROUPS - 1))];
  };

  const unsigned char* kbase = reinterpret_cast<const unsigned char*>(a.k) + (int64_t)h * a.k_sh * 2;
  const unsigned char* vbase = reinterpret_cast<const unsigned char*>(a.v) + (int64_t)h * a.v_sh * 2;
  const uint32_t k_sn2 = (uint32_t)(a.k_sn * 2), v_sn2 = (uint32_t)(a.v_sn * 2);
  const uint32_t k_ss2 = (uint32_t)(a.k_ss * 2), v_ss2 = (uint32_t)(a.v_ss * 2);

  // Per copy i of this wave: the lane's row within the tile, its source
  // chunks, and its byte offsets within the granule's K and V rows.
  auto copy_row = [&](int i) { return (wave * GPW + i) * RPG + lane / CPR; };
  auto k_chunk = [&](int i) { return (lane % CPR) ^ k_swz<CPR>(copy_row(i)); };
  auto v_chunk = [&](int i) { return (lane % CPR) ^ v_swz<CPR>(copy_row(i)); };
  uint32_t koff[GPW], voff[GPW];
#pragma unroll
  for (int i = 0; i < GPW; ++i) {
    koff[i] = (uint32_t)(copy_row(i) & 15) * k_ss2 + (uint32_t)(k_chunk(i) * 16);
    voff[i] = (uint32_t)(copy_row(i) & 15) * v_ss2 + (uint32_t)(v_chunk(i) * 16);
  }
  const bool all_dims = a.D == DP;
  const int kbuf0 = grp * STAGES, vbuf0 = grp * STAGES;  // this group's first K and V buffers

  const uint32_t k_dst0 = lds_addr(k_lds) + wave * (GPW * 1024);  // this wave's copy destinations
  const uint32_t v_dst0 = lds_addr(v_lds) + wave * (GPW * 1024);
  // The copies of one tile by this wave: per granule j its K and V
  // sources, whether every row is a key (the scalar-base form), and the
  // destinations.
  struct CopyPlan {
    const unsigned char* kb[GRW];
    const unsigned char* vb[GRW];
    int G[GRW];
    uint32_t kdst, vdst;
    int kt0;
    bool fast, live;
  };
  // Plans group tg's tile of step u (granules gv) into that group's K buffer
  // KS and V buffer VS; sets the tile's key mask (bit k: key k has K and V
  // rows). Nothing is copied past the last tile.
  auto plan_copies = [&](int u, int gv, int KS, int VS, uint64_t& vm, int tg) __attribute__((always_inline)) -> CopyPlan {
    CopyPlan cp;
    const int t = u * GROUPS + tg;
    cp.live = t < ntiles;
    cp.kt0 = key0 + t * kTileKeys;
    const uint32_t valid = ((uint32_t)__builtin_amdgcn_ballot_w64(gv >= 0) >> (4 * tg)) & 0xfu;  // granule j valid
    cp.fast = all_dims && cp.kt0 + kTileKeys <= kv_end && valid == 0xfu;
    cp.kdst = (tg * STAGES + KS) * TILEB;  // offsets from this wave's LDS bases (k_dst0, v_dst0)
    cp.vdst = (tg * STAGES + VS) * TILEB;
    const int gw0 = 4 * tg + ((wave * RW) >> 4);
#pragma unroll
    for (int j = 0; j < GRW; ++j) {
      const int G = __builtin_amdgcn_readlane(gv, gw0 + j);
      const uint32_t phys = (uint32_t)(G >> gshift), inb = (uint32_t)((G & gmask) << 4);
      cp.G[j] = G;
      cp.kb[j] = kbase + (uint64_t)phys * k_sn2 + inb * k_ss2;
      cp.vb[j] = vbase + (uint64_t)phys * v_sn2 + inb * v_ss2;
    }
    // Bit j of `valid` spread to bits 16j .. 16j + 15 (two 32-bit halves,
    // each a product with 0xffff of bits 16 apart).
    const uint32_t vl = cp.live ? valid : 0u;
    const uint32_t lo = ((vl & 1u) | ((vl & 2u) << 15)) * 0xffffu;
    const uint32_t hi = (((vl >> 2) & 1u) | ((vl & 8u) << 13)) * 0xffffu;
    vm = ((uint64_t)hi << 32) | lo;
    return cp;
  };
  // Issues copy i (one K and one V row group) of a plan. The LDS
  // destination is formed at the copy from this wave's two bases, passed
  // through an empty asm so the compiler cannot hoist every base + offset
  // sum out of the loop: held in scalar registers, those sums (one per
  // copy, stage and group) ran past the register file and were spilled to
  // vector-register lanes, a v_readlane per copy.
  auto copy_one = [&](const CopyPlan& cp, int i, auto fast) __attribute__((always_inline)) {
    const int j = i / CPGW;
    uint32_t kd = k_dst0, vd = v_dst0;
    asm volatile("" : "+s"(kd), "+s"(vd));
    kd += cp.kdst + i * 1024;
    vd += cp.vdst + i * 1024;
    if constexpr (decltype(fast)::value) {
      copy16_to_lds(cp.kb[j], koff[i], kd);
      copy16_to_lds(cp.vb[j], voff[i], vd);
    } else {
      const bool ok = cp.G[j] >= 0 && cp.kt0 + copy_row(i) < kv_end;
      const int ck = k_chunk(i), cv = v_chunk(i);
      const unsigned char* ks = (ok && ck * 8 < a.D) ? cp.kb[j] + koff[i] : kZeroRow + ck * 16;
      const unsigned char* vs = (ok && cv * 8 < a.D) ? cp.vb[j] + voff[i] : kZeroRow + cv * 16;
      copy16_to_lds(ks, kd);
      copy16_to_lds(vs, vd);
    }
  };
  // One branch per tile: the full-tile form's copies, or the masked form's.
  auto copy_all = [&](const CopyPlan& cp) __attribute__((always_inline)) {
    if (!cp.live) return;
    if (cp.fast) {
#pragma unroll
      for (int i = 0; i < GPW; ++i) copy_one(cp, i, Stage<1>{});
    } else {
#pragma unroll
      for (int i = 0; i < GPW; ++i) copy_one(cp, i, Stage<0>{});
    }
  };

  // Running sums of P come out of the PV products: lacc[b] = ones^T P^T, a
  // 16-row block of ones in place of V^T, so each lane holds the sum over
  // every key of its query column, four times (no VALU adds, no cross-lane
  // sum at the end). The sum is of the 2-byte P the output accumulates.
  // Softmax state per 16-row block: the reference maximum m_run (log2
  // domain), neg_m = -m_run (0 while m_run = -inf), and thr = (m_run +
  // slack) / scale, the raw-score maximum past which a tile rescales (-inf
  // while m_run = -inf). neg_m and thr change only on a rescale, so a tile
  // that does not rescale spends one compare per block on the check.
  f32x4_t oacc[QPW][NDB], lacc[QPW];
  float m_run[QPW], neg_m[QPW], thr[QPW];
#pragma unroll
  for (int b = 0; b < QPW; ++b) {
#pragma unroll
    for (int i = 0; i < NDB; ++i) oacc[b][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    lacc[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    m_run[b] = -INFINITY;
    neg_m[b] = 0.f;
    thr[b] = -INFINITY;
  }
  const uint32_t one2 = MM::pack2(1.f, 1.f);
  const uint4 ones = make_uint4(one2, one2, one2, one2);

  // This lane's operand read offsets within its group's stage 0. K: the A
  // row of key block kb is 32 (kb >> 1) + 4 (kb & 1) + krb, whose swizzle
  // equals krb's (the added terms leave the bits ks reads alone). V: rows
  // 32c + 4u + vr at head dims 16db + 4 tr_q, whose swizzle equals vr's.
  const int krb = 8 * (col >> 2) + (col & 3);
  int ka[NQF];
#pragma unroll
  for (int f = 0; f < NQF; ++f) ka[f] = kbuf0 * TILEB + krb * ROWB + (((4 * f + g) ^ k_swz<CPR>(krb)) << 4);
  const int tr_j = (lane & 15) >> 2, tr_q = lane & 3;
  const int vr = 8 * g + tr_j;
  uint32_t va[NDB];  // LDS byte addresses
#pragma unroll
  for (int db = 0; db < NDB; ++db)
    va[db] = lds_addr(v_lds) + vbuf0 * TILEB + vr * ROWB + ((tr_q & 1) << 3) +
             (((2 * db + (tr_q >> 1)) ^ v_swz<CPR>(vr)) << 4);
  const float cs = query_scale(a.scale_log2);  // the query carries the sign (query_sign)
  const float inv_cs = 1.f / cs;

  // QK^T and softmax of the tile in stage ST for the blocks in the mask
  // (bit b: block b; a Stage<mask> tag): packs P for the PV product.
  auto qk_softmax = [&](auto bm, int kt0, uint64_t vm, int ST, uint4 (&pb)[QPW][2]) __attribute__((always_inline)) {
    constexpr int BM = decltype(bm)::value;
    const unsigned char* kl = k_lds + ST * TILEB;
    // ---- S^T blocks: lane holds keys 32c + 8g + 4hh + i (kb = 2c + hh) of
    // query column `col` of each 16-row block b. Block kb + 1's K reads go
    // out before block kb's products; each read feeds QPW products.
    f32x4_t s[QPW][4];
    auto read_k = [&](int kb, uint4 (&kv)[NQF]) __attribute__((always_inline)) {
#pragma unroll
      for (int f = 0; f < NQF; ++f)
        kv[f] = *reinterpret_cast<const uint4*>(kl + ka[f] + (32 * (kb >> 1) + 4 * (kb & 1)) * ROWB);
    };
    uint4 kv[2][NQF];
    read_k(0, kv[0]);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      if (kb + 1 < 4) read_k(kb + 1, kv[(kb + 1) & 1]);
#pragma unroll
      for (int b = 0; b < QPW; ++b) s[b][kb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int f = 0; f < NQF; ++f)
#pragma unroll
        for (int b = 0; b < QPW; ++b)
          if ((BM >> b) & 1) s[b][kb] = MM::mfma(kv[kb & 1][f], qf[b][f], s[b][kb]);
      __builtin_amdgcn_sched_barrier(0);
    }

    // ---- masks (causal, invalid granules), online softmax, P packed for PV
    const bool full_wave = kt0 + kTileKeys - 1 <= wave_first && vm == ~0ull;
#pragma unroll
    for (int b = 0; b < QPW; ++b) {
      if (!((BM >> b) & 1)) continue;
      // PAIRED blocks lie apart, so each block tests its own first row.
      const bool full = PAIRED ? kt0 + kTileKeys - 1 <= blk_first[b] && vm == ~0ull : full_wave;
      float p[4][4];
      if (full) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) p[kb][i] = s[b][kb][i];
      } else {
        // Defined here, so the compiler cannot hoist this path's index
        // arithmetic above the branch into every full tile.
        int g8 = 8 * g;
        asm volatile("" : "+v"(g8));
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          const int k0 = 32 * (kb >> 1) + g8 + 4 * (kb & 1);  // within the tile
          const uint32_t bits = (uint32_t)(vm >> k0) & 0xfu;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bool vis = kt0 + k0 + i <= qpos[b] && ((bits >> i) & 1u);
            p[kb][i] = vis ? s[b][kb][i] : -INFINITY;
          }
        }
      }
      float mt = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) mt = fmaxf(mt, p[kb][i]);
      if (__builtin_amdgcn_ballot_w64(mt > thr[b]) != 0) {
        const float m_new = fmaxf(m_run[b], cross_group_max(mt) * cs);
        const float alpha = m_run[b] == -INFINITY ? 0.f : fast_exp2(m_run[b] - m_new);
        m_run[b] = m_new;
        neg_m[b] = m_new == -INFINITY ? 0.f : -m_new;
        thr[b] = m_new == -INFINITY ? -INFINITY : (m_new + kRescaleSlack) * inv_cs;
        lacc[b] *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db) oacc[b][db] *= alpha;
      }
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) p[kb][i] = fast_exp2(fmaf(p[kb][i], cs, neg_m[b]));
#pragma unroll
      for (int c = 0; c < 2; ++c)
        pb[b][c] = make_uint4(MM::pack2(p[2 * c][0], p[2 * c][1]), MM::pack2(p[2 * c][2], p[2 * c][3]),
                              MM::pack2(p[2 * c + 1][0], p[2 * c + 1][1]),
                              MM::pack2(p[2 * c + 1][2], p[2 * c + 1][3]));
    }
  };
  // O^T += V^T P^T (and the row sums) for the tile in stage ST, per 32-key
  // slice c; each V read feeds QPW products.
  auto pv = [&](auto bm, int ST, const uint4 (&pb)[QPW][2]) __attribute__((always_inline)) {
    constexpr int BM = decltype(bm)::value;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      uint4 vv[NDB];
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const uint2 lo = TrRead<T>::at(va[db] + ST * TILEB + (32 * c) * ROWB);
        const uint2 hi = TrRead<T>::at(va[db] + ST * TILEB + (32 * c + 4) * ROWB);
        vv[db] = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int b = 0; b < QPW; ++b)
          if ((BM >> b) & 1) oacc[b][db] = MM::mfma(vv[db], pb[b][c], oacc[b][db]);
#pragma unroll
      for (int b = 0; b < QPW; ++b)
        if ((BM >> b) & 1) lacc[b] = MM::mfma(ones, pb[b][c], lacc[b]);
      __builtin_amdgcn_sched_barrier(0);  // slice 1's V reads wait for slice 0's products
    }
  };

  // ---- pipeline, per group: the group's tiles of steps u + 1 .. u + STAGES
  // - 1 are copied while its tile of step u is computed. At step u: wait for
  // this wave's copies of its tile (later tiles' copies, 2 GPW per group
  // tile, may stay in flight; group 0 issues them for both groups, group 1
  // has none) and join the barrier (every wave's copies of it have landed and every
  // wave is done with the buffers of step u - 1), start the tile of step
  // u + STAGES - 1 in them, read the granules of the step after it,
  // compute. Buffers of step u: u % STAGES.
  auto wait_step = [&](int u) {
    const int later = ntg - 1 - u;  // this group's tiles after step u whose copies may be in flight
    if constexpr (STAGES >= 4)
      if (later >= 2) return wait_and_barrier<4 * GPW * GROUPS>();
    if constexpr (STAGES >= 3)
      if (later >= 1) return wait_and_barrier<2 * GPW * GROUPS>();
    wait_and_barrier<0>();
  };
  // The copies of step u into buffers ST: with two groups, group 0 copies
  // both groups' tiles and group 1 only derives its tile's mask, so group 1
  // starts computing right after the barrier while group 0 issues.
  auto issue_step = [&](int u, int gv, int ST, uint64_t& vm_own) __attribute__((always_inline)) {
    if constexpr (GROUPS == 1) {
      copy_all(plan_copies(u, gv, ST, ST, vm_own, 0));
    } else {
      uint64_t vm_other;
      if (grp == 0) {
        copy_all(plan_copies(u, gv, ST, ST, vm_own, 0));
        copy_all(plan_copies(u, gv, ST, ST, vm_other, 1));
      } else {
        (void)plan_copies(u, gv, ST, ST, vm_own, 1);
      }
    }
  };
  uint64_t vm[STAGES];
  int e = tile_granules(0);
  static_for<0, STAGES - 1>([&](auto sc) {
    constexpr int SI = decltype(sc)::value;
    vm[SI] = 0;
    if (SI < nsteps) {
      issue_step(SI, e, SI, vm[SI]);
      if (SI + 1 < nsteps) e = tile_granules(SI + 1);
    }
  });
  // Steps [u_lo, u_hi) with the blocks of mask bm (a Stage<mask> tag).
  auto run_steps = [&](auto bm, int u_lo, int u_hi) __attribute__((always_inline)) {
    for (int u0 = u_lo - u_lo % STAGES; u0 < u_hi; u0 += STAGES) {
      static_for<0, STAGES>([&](auto sc) {
        constexpr int SI = decltype(sc)::value;
        constexpr int SN = (SI + STAGES - 1) % STAGES;  // buffers of step u + STAGES - 1
        const int u = u0 + SI;
        if (u < u_lo || u >= u_hi) return;
        wait_step(u);
        const int un = u + STAGES - 1;
        if (un < nsteps) {
          issue_step(un, e, SN, vm[SN]);
          if (un + 1 < nsteps) e = tile_granules(un + 1);
        }
        const int kt0 = key0 + (u * GROUPS + grp) * kTileKeys;
        if (u < ntg && wave_active && kt0 <= wave_last) {
          uint4 pb[QPW][2];
          qk_softmax(bm, kt0, vm[SI], SI, pb);
          pv(bm, SI, pb);
        }
      });
    }
  };
  if constexpr (PAIRED) {
    // Block 0's rows come first. The steps whose tile (of this wavefront's
    // group) reaches them run both blocks, the rest block 1 alone, in two
    // loops: one loop with a branch between the two bodies made the compiler
    // spill registers. Where block 1 has no rows, every step runs both (its
    // rows past the chunk are computed and never stored).
    int u_split = nsteps;
    if (rb[1] < a.T) {
      const int f = rb[0] < a.T ? (blk_last[0] - key0) / kTileKeys - grp : -1;
      u_split = f >= 0 ? min(nsteps, f / GROUPS + 1) : 0;
    }
    run_steps(Stage<3>{}, 0, u_split);
    run_steps(Stage<2>{}, u_split, nsteps);
  } else {
    run_steps(Stage<(1 << QPW) - 1>{}, 0, nsteps);
  }


  // ---- group 1 hands its state to group 0 through the drained tile
  // buffers: unnormalised outputs in the K buffers, (max, partial sum) in the
  // V buffers, lane-major so the writes and reads are conflict-free.
  if constexpr (GROUPS == 2) {
    constexpr int OITEMS = QPW * 4 * NDB;  // output floats per lane
    static_assert(OITEMS * 64 * WAVES * 4 <= KBUFS * TILEB, "group 1's outputs fit the K buffers");
    static_assert(2 * QPW * 64 * WAVES * 4 <= VBUFS * TILEB, "group 1's (max, sum) fit the V buffers");
    float* xo = reinterpret_cast<float*>(k_lds) + wave * (OITEMS * 64) + lane;
    float* xm = reinterpret_cast<float*>(v_lds) + wave * (2 * QPW * 64) + lane;
    wait_and_barrier<0>();  // every wave is done with the tile buffers
    if (grp == 1) {
#pragma unroll
      for (int b = 0; b < QPW; ++b) {
        xm[(2 * b) * 64] = m_run[b];
        xm[(2 * b + 1) * 64] = lacc[b][0];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int i = 0; i < 4; ++i) xo[((b * NDB + db) * 4 + i) * 64] = oacc[b][db][i];
      }
    }
    __syncthreads();
    if (grp == 1) return;
#pragma unroll
    for (int b = 0; b < QPW; ++b) {
      const float m1 = xm[(2 * b) * 64], l1 = xm[(2 * b + 1) * 64];
      const float m_new = fmaxf(m_run[b], m1);
      const float a0 = m_run[b] == -INFINITY ? 0.f : fast_exp2(m_run[b] - m_new);
      const float a1 = m1 == -INFINITY ? 0.f : fast_exp2(m1 - m_new);
      m_run[b] = m_new;
      lacc[b][0] = lacc[b][0] * a0 + l1 * a1;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          oacc[b][db][i] = oacc[b][db][i] * a0 + xo[((b * NDB + db) * 4 + i) * 64] * a1;
    }
  }

  // ---- normalise and store (as paged_prefill_mfma)
#pragma unroll
  for (int b = 0; b < QPW; ++b) {
    const float l = lacc[b][0];
    if (qi[b] >= a.T) continue;
    if (a.part_keys > 0) {
      const int np = (a.start + qi[b] + a.part_keys) / a.part_keys;
      if (part >= np) continue;
      if (np > 1) {
        const size_t slot = ((size_t)qi[b] * a.H + h) * a.max_parts + part;
        if (g == 0) a.ws_ml[slot] = make_float2(m_run[b], l);
        float* wa = a.ws_acc + slot * a.D;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const int d0 = 16 * db + 4 * g;
          if (d0 >= a.D) continue;
          *reinterpret_cast<float4*>(wa + d0) =
              make_float4(oacc[b][db][0], oacc[b][db][1], oacc[b][db][2], oacc[b][db][3]);
        }
        continue;
      }
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    T* orow = reinterpret_cast<T*>(a.out) + (int64_t)qi[b] * a.o_st + (int64_t)h * a.o_sh;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int d0 = 16 * db + 4 * g;
      if (d0 >= a.D) continue;
      uint2 w;
      w.x = MM::pack2(oacc[b][db][0] * inv, oacc[b][db][1] * inv);
      w.y = MM::pack2(oacc[b][db][2] * inv, oacc[b][db][3] * inv);
      *reinterpret_cast<uint2*>(orow + d0) = w;
    }
  }
}

// Workgroups of kernel `fn` (threads each) resident per CU at once.
static int resident_per_cu(const void* fn, int threads) {
  int n = 0;
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, 0) == hipSuccess ? n : 0;
}

// Whether paged_prefill_tr takes this call: power-of-two blocks of at least
// 16 keys, D a multiple of 8, 16-byte aligned rows, and the 32-bit offsets it
// forms in range (granule indices, block strides, in-block row offsets).
static bool tr_eligible(const PrefillArgs& a) {
  if (a.s_shift < 4 || a.D % 8 != 0) return false;
  const int64_t lim = (int64_t)1 << 31;
  if ((a.N << (a.s_shift - 4)) >= lim) return false;
  for (int64_t sn : {a.k_sn, a.v_sn})
    if (sn < 0 || sn * 2 >= ((int64_t)1 << 32)) return false;
  for (int64_t ss : {a.k_ss, a.v_ss})
    if (ss < 0 || (int64_t)a.S * ss * 2 >= lim || (ss * 2) % 16 != 0) return false;
  for (int64_t sx : {a.k_sn, a.v_sn, a.k_sh, a.v_sh})
    if ((sx * 2) % 16 != 0) return false;
  return (reinterpret_cast<uintptr_t>(a.k) % 16) == 0 && (reinterpret_cast<uintptr_t>(a.v) % 16) == 0;
}

template <typename T, int DP, int WAVES, int QPW, int STAGES, int GROUPS, bool PAIRED = false>
hipError_t launch_tr_cfg(const PrefillArgs& a, hipStream_t stream) {
  constexpr int QB = 16 * QPW * WAVES;
  constexpr int HB = 16 * WAVES;
  constexpr int NT = 64 * WAVES * GROUPS;
  const int64_t wgs = (PAIRED ? (((int64_t)a.T + HB - 1) / HB + 1) / 2 : ((int64_t)a.T + QB - 1) / QB) * a.H;
  const void* fn = reinterpret_cast<const void*>(&paged_prefill_tr<T, DP, WAVES, QPW, STAGES, GROUPS, PAIRED>);
  static const int per_cu = resident_per_cu(fn, NT);
  PrefillArgs b = a;
  const bool split = a.part_keys > 0;
  b.pair_round = (!split && per_cu == 2 && (a.H & 7) == 0 && a.cus % 8 == 0 && wgs > a.cus &&
                  wgs <= 2 * a.cus)
                     ? a.cus / 8 : 0;
  const dim3 grid((unsigned)wgs, split ? (unsigned)a.max_parts : 1u);
  hipLaunchKernelGGL((paged_prefill_tr<T, DP, WAVES, QPW, STAGES, GROUPS, PAIRED>), grid, dim3(NT), 0, stream, b);
  return hipGetLastError();
}

// MINIVLLM_HIP_PREFILL_TR (read on every call) overrides the choice below for
// tuning and tests: 0 takes paged_prefill_mfma; otherwise its decimal digits
// set paged_prefill_tr's paired rows (ten thousands), groups minus one
// (thousands), wavefronts per group, 16-row query blocks per wavefront and
// tiles in flight per group (412, 422, 812, 1412, 1422 or 11422). -1: unset.
int prefill_tr_mode() {
  const char* e = std::getenv("MINIVLLM_HIP_PREFILL_TR");
  return e && *e ? std::atoi(e) : -1;
}

// paged_prefill_tr configuration for a call, measured on MI355X (bf16,
// D = 128, S = 16, 16 heads unless noted):
//   * 11422 (1422 with paired rows: one workgroup per pair of 64-row half
//     tiles) when those workgroups fill at least 7/8 of the CUs in one
//     round: every workgroup then holds the same work. 2048 rows after
//     2048: 68.2 against 71.1 us for 1422; at 0: 35.5 (1412: 38.0);
//     after 512: 43.6 (1422: 47.6); after 4096 and 8192: 98.5 / 160.2
//     (1422: 102.1 / 163.6); 8 heads, 4096 rows at 0: 58.0 (1412: 58.5,
//     1422: 67.9), after 4096: 121.7 (1422: 130.7); 32 heads, 1024 rows
//     at 0 and after 1024: 24.5 / 40.2 (412: 25.1, 1422: 42.0). A grid
//     that fills 3/4 of the CUs leaves them idle all the same, and there
//     the others win (1536 rows after 1536: 66.8 against 60.3 for 412);
//   * 1422 (two groups of four 32-row wavefronts per 128-row query tile,
//     one workgroup per CU): chunks after a prefix at least as long whose
//     128-row tiles fill the CUs (2048 rows after 2048: 72-80 us; 412:
//     77-87), and chunks whose 128-row tiles take more than one round of the
//     CUs while the mean tile attends to at least 20 key tiles (4096 rows at
//     0: 85 us, 412: 94; 2560 rows: 48 / 52.5; 8192 rows: 296 / 348; 3072
//     after 1024: 85 / 90). Below 20 the two groups' hand-over and the
//     one-per-CU grid lose (1024 rows at 0 with 64 heads: 46.6 / 43.3);
//   * 1412 (two groups of four 16-row wavefronts per 64-row tile): grids of
//     64-row tiles that leave CUs empty, where splitting each workgroup's keys
//     over two groups halves its serial chain (512 rows at 0: 13.5 us; 412:
//     14.5), and first chunks (start 0) whose 64-row tiles take up to two
//     rounds of the CUs (1536 rows: 26.8 against 31.3 for 412; 8 heads,
//     3072 rows: 40.5 against 54.1);
//   * with the keys split over workgroups (the cost model sizes partitions
//     for 64-row tiles): 1422 when its 128-row tiles times the partitions
//     fill the CUs and a partition holds at least 32 key tiles (512 rows
//     after 16 384: 83 against 98 us for 412; after 8192: 51.7 / 58.4; 32
//     heads, 256 after 8192: 53 / 58), else 412 (256 after 4096: 27 against
//     29 for 1422; 32 heads, 512 after 2048, 19-tile partitions: 45.6 /
//     48.6), whose two-group hand-over does not pay on short partitions;
//   * 412 (two workgroups of four 16-row wavefronts per CU) otherwise, and
//     for chunks whose keys fit one tile (64 rows at 0, 16 and 32 heads:
//     8.4-8.5 against 9.4-9.6 us for 1412).
int prefill_tr_choice(const PrefillArgs& a) {
  const int forced = prefill_tr_mode();
  if (forced >= 0) return forced;
  const int64_t wgs128 = ((int64_t)a.T + 127) / 128 * a.H, wgs64 = ((int64_t)a.T + 63) / 64 * a.H;
  const int64_t wgs_paired = (((int64_t)a.T + 63) / 64 + 1) / 2 * a.H;
  if (a.part_keys > 0)
    return wgs128 * a.max_parts >= a.cus && a.part_keys >= 32 * kTileKeys ? 1422 : 412;
  if (a.start + a.T <= kTileKeys) return 412;  // one key tile: a second group would idle
  if (wgs_paired <= a.cus && 8 * wgs_paired >= 7 * (int64_t)a.cus) return 11422;
  const int64_t mean_keys = (int64_t)a.start + a.T / 2;  // keys the mean query tile attends to
  if (wgs128 >= a.cus && (a.start >= a.T || (wgs128 > a.cus && mean_keys >= 20 * kTileKeys))) return 1422;
  if (wgs64 <= a.cus || (a.start == 0 && wgs64 <= 2 * (int64_t)a.cus)) return 1412;
  return 412;
}

template <typename T, int DP>
hipError_t launch_tr(const PrefillArgs& a, int mode, hipStream_t stream) {
  switch (mode) {
    case 422: return launch_tr_cfg<T, DP, 4, 2, 2, 1>(a, stream);
    case 812: return launch_tr_cfg<T, DP, 8, 1, 2, 1>(a, stream);
    case 1412: return launch_tr_cfg<T, DP, 4, 1, 2, 2>(a, stream);
    case 1422: return launch_tr_cfg<T, DP, 4, 2, 2, 2>(a, stream);
    case 11422: return launch_tr_cfg<T, DP, 4, 2, 2, 2, true>(a, stream);
    default: return launch_tr_cfg<T, DP, 4, 1, 2, 1>(a, stream);  // 412
  }
}

template <typename T, int DP, int WAVES>
hipError_t launch_waves(const PrefillArgs& a, hipStream_t stream) {
  if constexpr (sizeof(T) == 2 && (DP == 64 || DP == 128) && WAVES == 4) {
    if (tr_eligible(a)) {
      const int mode = prefill_tr_choice(a);
      if (mode != 0) return launch_tr<T, DP>(a, mode, stream);
    }
  }
  constexpr int QB = 16 * WAVES;
  const void* fn = reinterpret_cast<const void*>(&paged_prefill_mfma<T, DP, WAVES, 1>);
  static const int per_cu = resident_per_cu(fn, 64 * WAVES);
  const int64_t wgs = ((int64_t)a.T + QB - 1) / QB * a.H;
  // Measured on MI355X: with two workgroups per CU and a grid that is
  // resident at once, pairing long with short query tiles per CU cuts the
  // 2048-row chunks by 8-19%. With one per CU (fp32 and the 256-wide bf16 /
  // f16 tiles fill the LDS) the grid runs in dynamic rounds, where the
  // longest-first order is better (the pairing cost fp32 16-33%).
  // Split keys add a grid dimension of partitions (the pairing assumes one
  // partition per query tile and is off then).
  PrefillArgs b = a;
  const bool split = a.part_keys > 0;
  b.pair_round = (!split && per_cu == 2 && (a.H & 7) == 0 && a.cus % 8 == 0 && wgs > a.cus &&
                  wgs <= 2 * a.cus)
                     ? a.cus / 8 : 0;
  hipLaunchKernelGGL((paged_prefill_mfma<T, DP, WAVES, 1>),
                     dim3((unsigned)wgs, split ? (unsigned)a.max_parts : 1u), dim3(64 * WAVES), 0, stream, b);
  return hipGetLastError();
}

template <typename T, int DP>
hipError_t launch_dp(const PrefillArgs& a, int waves, int qpw, hipStream_t stream) {
  (void)qpw;  // one 16-row block per wavefront (see launch_paged_prefill)
  return waves == 4 ? launch_waves<T, DP, 4>(a, stream) : launch_waves<T, DP, 2>(a, stream);
}

}  // namespace

int prefill_head_dim_bucket(int two_byte, int D) {
  if (D <= 32) return 32;
  if (D <= 64) return 64;
  if (D <= 128) return 128;
  if (two_byte && D <= 256) return 256;
  return 0;
}

// Measured on MI355X (bf16, H=16, D=128; chunks of 406-2048 rows after
// prefixes of 0-2048): four wavefronts of one 16-row block each beat two
// blocks per wavefront (which holds one wavefront per SIMD, so MFMA and
// softmax work cannot overlap across wavefronts) and two- or eight-wavefront
// workgroups, so only QPW == 1 is instantiated.
hipError_t launch_paged_prefill(const PrefillArgs& a, int dtype, int dp, int waves, int qpw,
                                hipStream_t stream) {
  if (dtype == MGI_BF16) {
    switch (dp) {
      case 32: return launch_dp<bf16_t, 32>(a, waves, qpw, stream);
      case 64: return launch_dp<bf16_t, 64>(a, waves, qpw, stream);
      case 128: return launch_dp<bf16_t, 128>(a, waves, qpw, stream);
      case 256: return launch_dp<bf16_t, 256>(a, waves, qpw, stream);
    }
  } else if (dtype == MGI_F16) {
    switch (dp) {
      case 32: return launch_dp<f16_t, 32>(a, waves, qpw, stream);
      case 64: return launch_dp<f16_t, 64>(a, waves, qpw, stream);
      case 128: return launch_dp<f16_t, 128>(a, waves, qpw, stream);
      case 256: return launch_dp<f16_t, 256>(a, waves, qpw, stream);
    }
  } else if (dtype == MGI_F32) {
    switch (dp) {
      case 32: return launch_dp<float, 32>(a, waves, 1, stream);
      case 64: return launch_dp<float, 64>(a, waves, 1, stream);
      case 128: return launch_dp<float, 128>(a, waves, 1, stream);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace mgi
