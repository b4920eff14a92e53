// paged_decode.hip -- paged decode attention for gfx950 (CDNA4, wave64).
//
// Semantics follow paged_attention_batch_online_v1
// (minivllm/paged_attention_batch.py:121-278) and the Triton v0 kernel
// (minivllm/triton_paged_decode.py:29-99): for each (sequence b, head h)
//   out = softmax(scale * q . K^T) V  over the ctx_b valid tokens reached
// through block_tables[b, 0 : ceil(ctx_b / S)]. Table entries past the
// context and pool slots past the context are never dereferenced.
//
// Fast path (fold_chunk, run by paged_decode_fast_bal or paged_decode_fast):
// a wavefront owns HPW = 64/LPH heads and streams a run of blocks of one
// sequence. LPH lanes share a head row, each lane owning 8 elements of
// head_dim, so one 16-byte load instruction of the wave reads a contiguous
// run of HPW head rows of one token (1 KiB for bf16, D=128). Per step the
// wave issues TOK tokens of K and V loads up front (32 KiB in flight per wave
// for bf16, TOK=16; non-temporal, as every byte is read once), then forms the
// TOK scores with packed 16-bit dot products and a DPP all-reduce inside each
// row of LPH lanes, and folds the step into an fp32 online softmax kept in
// the log2 domain. Decode attention is HBM-bound (~1 flop/byte), so there is
// no MFMA and no LDS staging: every lane loads exactly the bytes it consumes.
//
// Work split: paged_decode_fast_bal deals the blocks of all sequences out to
// a fixed number of wavefronts, most of them as each wave's own claim and the
// rest as small claims that waves draw by ticket once their own is done, so
// faster XCDs take more (the automatic choice); paged_decode_fast cuts each
// context into partitions of part_tokens tokens.
// A sequence whose work is split writes (max, sum, unnormalised output)
// partials that paged_decode_merge combines:
//   M = max_p m_p,  L = sum_p l_p 2^(m_p - M),  O = sum_p O_p 2^(m_p - M) / L.
//
// Fused KV append (mgi_paged_decode_append, fast path): the wavefront of a
// head group that streams sequence b's last block first copies that head
// group's slice of row b of the new K/V to pool slot slot_mapping[b], then
// streams the block; it reads the slot after writing it, in program order,
// so attention sees exactly the pool a separate append would have left. A
// row whose sequence has no blocks is copied by a wavefront of its own.
//
// The fast path covers bf16, f16 (the same lane layout, v_dot2_f32_f16) and
// f32. Generic path (paged_decode_generic): any strides, head_dim up to 512,
// any block size, f32/bf16/f16; one wavefront per (b, h), one token at a time.
#include "mgi_common.h"
#include "mgi_internal.h"
#include "minivllm_hip.h"

namespace mgi {

// ------------------------------------------------------------ lane layout
// A lane owns 8 elements of one head row.
//   2-byte types: d = 8*sub + i                       (one 16-byte load)
//   f32:          d = 4*sub + i            (i < 4)    (two 16-byte loads, each
//                 d = D/2 + 4*sub + i - 4  (i >= 4)    contiguous across lanes)
template <typename T> struct Layout;
template <> struct Layout<bf16_t> {
  static constexpr int kLoads = 1;
  __device__ static int load_off(int sub, int /*D*/, int /*j*/) { return 8 * sub; }
  __device__ static int elem(int sub, int /*D*/, int i) { return 8 * sub + i; }
};
template <> struct Layout<f16_t> : Layout<bf16_t> {};
template <> struct Layout<float> {
  static constexpr int kLoads = 2;
  __device__ static int load_off(int sub, int D, int j) { return j * (D >> 1) + 4 * sub; }
  __device__ static int elem(int sub, int D, int i) { return (i >> 2) * (D >> 1) + 4 * sub + (i & 3); }
};

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Element i (0..7) of a lane's raw fragment as f32.
template <typename T>
__device__ __forceinline__ float frag_elem(const uint4 (&r)[Layout<T>::kLoads], int i);
template <>
__device__ __forceinline__ float frag_elem<bf16_t>(const uint4 (&r)[1], int i) {
  const uint32_t w = (i >> 1) == 0 ? r[0].x : (i >> 1) == 1 ? r[0].y : (i >> 1) == 2 ? r[0].z : r[0].w;
  return (i & 1) ? bf16_hi(w) : bf16_lo(w);
}
template <>
__device__ __forceinline__ float frag_elem<f16_t>(const uint4 (&r)[1], int i) {
  const uint32_t w = (i >> 1) == 0 ? r[0].x : (i >> 1) == 1 ? r[0].y : (i >> 1) == 2 ? r[0].z : r[0].w;
  return f16_to_f32((uint16_t)((i & 1) ? (w >> 16) : (w & 0xffffu)));
}
template <>
__device__ __forceinline__ float frag_elem<float>(const uint4 (&r)[2], int i) {
  const uint4& x = r[i >> 2];
  const uint32_t w = (i & 3) == 0 ? x.x : (i & 3) == 1 ? x.y : (i & 3) == 2 ? x.z : x.w;
  return __uint_as_float(w);
}

// Query fragment: packed 16-bit pairs (exact) for bf16 and f16, f32 values
// for f32. The 2-byte types dot with v_dot2_f32_bf16 / v_dot2_f32_f16 (f32
// accumulate; the products of two 16-bit values are exact in f32).
template <typename T> struct QFrag;
template <typename T>
struct QFrag16 {
  uint32_t w[4];
  __device__ static __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    if constexpr (sizeof(T) == 2 && __is_same(T, bf16_t))
      return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                             __builtin_bit_cast(bf16x2, b), c, false);
    else
      return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c,
                                    false);
  }
  __device__ __forceinline__ float dot(const uint4 (&k)[1]) const {
    float d = 0.f;
    d = dot2(w[0], k[0].x, d);
    d = dot2(w[1], k[0].y, d);
    d = dot2(w[2], k[0].z, d);
    d = dot2(w[3], k[0].w, d);
    return d;
  }
  __device__ __forceinline__ void load(const T* row, int64_t sd, int sub, int D) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(row);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = p[(int64_t)Layout<T>::elem(sub, D, 2 * j) * sd];
      const uint32_t hi = p[(int64_t)Layout<T>::elem(sub, D, 2 * j + 1) * sd];
      w[j] = lo | (hi << 16);
    }
  }
  __device__ __forceinline__ void zero() { w[0] = w[1] = w[2] = w[3] = 0u; }
};
template <> struct QFrag<bf16_t> : QFrag16<bf16_t> {};
template <> struct QFrag<f16_t> : QFrag16<f16_t> {};
template <> struct QFrag<float> {
  float f[8];
  __device__ __forceinline__ float dot(const uint4 (&k)[2]) const {
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) d = fmaf(f[i], frag_elem<float>(k, i), d);
    return d;
  }
  __device__ __forceinline__ void load(const float* row, int64_t sd, int sub, int D) {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = row[(int64_t)Layout<float>::elem(sub, D, i) * sd];
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = 0.f;
  }
};

template <typename T>
__device__ __forceinline__ int clamp_ctx(const DecodeArgs& a, int b) {
  const int64_t c = a.cl ? load_index(a.cl, a.cl_i64, (int64_t)b * a.cl_s) : a.ctx_base + b + 1;
  const int64_t max_ctx = (int64_t)a.M * a.S;
  return (int)(c < 0 ? 0 : (c > max_ctx ? max_ctx : c));
}

// Stores a lane's 8 output elements (acc * inv) into out[b, h, :].
template <typename T>
__device__ __forceinline__ void store_out(const DecodeArgs& a, int b, int h, int sub,
                                          const float (&acc)[8], float inv) {
  T* orow = reinterpret_cast<T*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    Elem<T>::store(orow + (int64_t)Layout<T>::elem(sub, a.D, i) * a.o_sd, acc[i] * inv);
}

// ------------------------------------------------------------- fast kernel

// Largest number of S-token blocks one chunk of a wave's work may span: the
// chunk's block-table entries are held one per lane in two VGPRs.
constexpr int kMaxBlocksPerPart = 128;

// Raw K and V fragments of TOK consecutive tokens of one block.
template <typename T, int TOK>
struct Step {
  uint4 k[TOK][Layout<T>::kLoads];
  uint4 v[TOK][Layout<T>::kLoads];
};

// Byte offsets of this lane's loads inside one token row of the pool.
template <typename T>
__device__ __forceinline__ void row_offsets(const DecodeArgs& a, int h, int sub, bool lane_ok,
                                            uint32_t (&koff)[Layout<T>::kLoads],
                                            uint32_t (&voff)[Layout<T>::kLoads]) {
  constexpr int EB = (int)sizeof(T);
#pragma unroll
  for (int j = 0; j < Layout<T>::kLoads; ++j) {
    koff[j] = lane_ok ? (uint32_t)(((int64_t)h * a.k_sh + Layout<T>::load_off(sub, a.D, j)) * EB) : 0u;
    voff[j] = lane_ok ? (uint32_t)(((int64_t)h * a.v_sh + Layout<T>::load_off(sub, a.D, j)) * EB) : 0u;
  }
}

template <typename T>
__device__ __forceinline__ void load_query(const DecodeArgs& a, int b, int h, int sub, bool lane_ok,
                                           QFrag<T>& q) {
  q.zero();
  if (lane_ok)
    q.load(reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh, a.q_sd, sub,
           a.D);
}

// Fused append, in two halves so their latencies overlap the caller's
// loads: append_load issues this lane's loads of piece j (0, and 1 for f32)
// of head h of row b of the new K and V; append_store writes a piece to pool
// slot `slot`. append_fence keeps every later load of this wavefront behind
// the stores in the compiler's order; the hardware keeps a wavefront's
// accesses to one address in order.
template <typename T>
__device__ __forceinline__ void append_load(const DecodeArgs& a, int b, int h, int sub, int j, uint4& kf,
                                            uint4& vf) {
  constexpr int EB = (int)sizeof(T);
  const int o = Layout<T>::load_off(sub, a.D, j) * EB;
  kf = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(a.kn) +
                                       ((int64_t)b * a.kn_sb + (int64_t)h * a.kn_sh) * EB + o);
  vf = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(a.vn) +
                                       ((int64_t)b * a.vn_sb + (int64_t)h * a.vn_sh) * EB + o);
}
template <typename T>
__device__ __forceinline__ void append_store(const DecodeArgs& a, int64_t slot, int h, int sub, int j,
                                             const uint4& kf, const uint4& vf) {
  constexpr int EB = (int)sizeof(T);
  const int64_t blk = slot / a.S, off = slot - blk * (int64_t)a.S;
  const int o = Layout<T>::load_off(sub, a.D, j) * EB;
  *reinterpret_cast<uint4*>(reinterpret_cast<char*>(a.kw) +
                            (blk * a.k_sn + off * a.k_ss + (int64_t)h * a.k_sh) * EB + o) = kf;
  *reinterpret_cast<uint4*>(reinterpret_cast<char*>(a.vw) +
                            (blk * a.v_sn + off * a.v_ss + (int64_t)h * a.v_sh) * EB + o) = vf;
}
__device__ __forceinline__ bool append_slot_ok(const DecodeArgs& a, int64_t slot) {
  return slot >= 0 && slot < a.N * (int64_t)a.S;
}
__device__ __forceinline__ void append_fence() { __atomic_signal_fence(__ATOMIC_SEQ_CST); }

// The fused append of one row in one go (rows of sequences with no blocks).
template <typename T, bool FULL>
__device__ __forceinline__ void append_row(const DecodeArgs& a, int b, int h, int sub, bool lane_ok) {
  const int64_t slot = load_index(a.slots, a.sl_i64, (int64_t)b * a.sl_s);
  if (!append_slot_ok(a, slot)) return;  // uniform
  if (FULL || lane_ok) {
#pragma unroll
    for (int j = 0; j < Layout<T>::kLoads; ++j) {
      uint4 kf, vf;
      append_load<T>(a, b, h, sub, j, kf, vf);
      append_store<T>(a, slot, h, sub, j, kf, vf);
    }
  }
  append_fence();
}

// Folds the tokens of blocks [blk_begin, blk_end) of sequence b, clipped to
// its context ctx, into the wave's online-softmax state (m, l, acc); the
// chunk spans at most kMaxBlocksPerPart blocks. Scores live in the log2
// domain.
template <typename T, int LPH, int TOK, bool FULL>
__device__ __forceinline__ void fold_chunk(const DecodeArgs& a, int b, int h, int lane, bool lane_ok,
                                            const QFrag<T>& q,
                                            const uint32_t (&koff)[Layout<T>::kLoads],
                                            const uint32_t (&voff)[Layout<T>::kLoads],
                                            int blk_begin, int blk_end, int ctx, float& m, float& l,
                                            float (&acc)[8]) {
  constexpr int NL = Layout<T>::kLoads;
  constexpr int EB = (int)sizeof(T);
  const int S = a.S;
  const char* kl = reinterpret_cast<const char*>(a.k);
  const char* vl = reinterpret_cast<const char*>(a.v);
  const int64_t k_row = a.k_ss * EB, v_row = a.v_ss * EB;
  const int steps_per_blk = S / TOK;
  const int64_t bt_row = (int64_t)b * a.bt_sb;

  {
    const int c0 = blk_begin;
    const int t_begin = c0 * S;  // a multiple of S
    const int t_end = min(ctx, blk_end * S);
    if (t_end <= t_begin) return;  // uniform over the wave
    const int nsteps = (t_end - t_begin + TOK - 1) / TOK;
    const int nblk = (t_end - t_begin + S - 1) / S;  // <= kMaxBlocksPerPart

    // Lane j holds the chunk's physical block ids j (phys_lo) and 64 + j
    // (phys_hi); -1 marks an out-of-range entry (masked) or no block.
    int phys_lo = -1, phys_hi = -1;
    if (lane < nblk) {
      const int64_t e = load_index(a.bt, a.bt_i64, bt_row + (int64_t)(c0 + lane) * a.bt_sm);
      phys_lo = (e >= 0 && e < a.N) ? (int)e : -1;
    }
    if (64 + lane < nblk) {
      const int64_t e = load_index(a.bt, a.bt_i64, bt_row + (int64_t)(c0 + 64 + lane) * a.bt_sm);
      phys_hi = (e >= 0 && e < a.N) ? (int)e : -1;
    }
    // The chunk holding the sequence's last token writes the fused append's
    // row: its loads go out beside the table entries', its stores just before
    // the loads of the chunk's last step, which reads the new token. Stores
    // count in the same in-order wait counter as loads, so stores issued
    // earlier would hold up the waits of the steps in between: at B=256,
    // 32 heads, stores before step 1 cost 8.7 us over decode alone, stores
    // before the last step 5.7 (the append kernel and its launch 6.3); at
    // B=64, 3.8 against 1.6 (4.4).
    const bool tail = a.kw != nullptr && t_end == ctx;
    const int asub = lane % LPH;
    const bool aok = FULL || lane_ok;
    uint4 ak0, av0, ak1, av1;
    int64_t aslot = -1;
    if (tail) {
      if (aok) append_load<T>(a, b, h, asub, 0, ak0, av0);
      if (aok && NL == 2) append_load<T>(a, b, h, asub, 1, ak1, av1);
      aslot = load_index(a.slots, a.sl_i64, (int64_t)b * a.sl_s);
    }
    auto append_stores = [&]() {
      if (!tail) return;
      if (append_slot_ok(a, aslot) && aok) {
        append_store<T>(a, aslot, h, asub, 0, ak0, av0);
        if (NL == 2) append_store<T>(a, aslot, h, asub, 1, ak1, av1);
      }
      append_fence();
    };

    // Issues the K/V loads of step s and returns its number of valid tokens
    // (0 past the chunk or for a masked block). Every iteration issues the
    // same loads, with no branch around them; a step past the chunk points
    // every lane at the same 16 bytes of the last step's first row (one line
    // per wave: the streaming loads are non-temporal, so re-reading the whole
    // last step would fetch it from HBM again).
    auto issue = [&](int s, Step<T, TOK>& st) -> int {
      if (s == nsteps - 1) append_stores();
      const bool past = s >= nsteps;
      const int sc = past ? nsteps - 1 : s;
      const int rel = sc / steps_per_blk;
      const int off = (sc - rel * steps_per_blk) * TOK;
      const int phys = rel < 64 ? __builtin_amdgcn_readlane(phys_lo, rel)
                                : __builtin_amdgcn_readlane(phys_hi, rel - 64);
      const int nvalid = past ? 1 : min(TOK, t_end - (t_begin + sc * TOK));
      const int64_t pb = phys >= 0 ? phys : 0;  // a masked block is read from block 0, never used
      const auto krs = make_rsrc(kl + (pb * a.k_sn + (int64_t)off * a.k_ss) * EB);
      const auto vrs = make_rsrc(vl + (pb * a.v_sn + (int64_t)off * a.v_ss) * EB);
      // Tokens past the context re-read the last valid token (never a slot
      // past the context) and are masked out of the softmax.
#pragma unroll
      for (int t = 0; t < TOK; ++t) {
        const uint32_t so = (uint32_t)((t < nvalid ? t : nvalid - 1) * k_row);
#pragma unroll
        for (int j = 0; j < NL; ++j) {
          if (FULL || lane_ok) st.k[t][j] = buffer_load16(krs, past ? 0u : koff[j], so);
          else st.k[t][j] = make_uint4(0u, 0u, 0u, 0u);
        }
      }
#pragma unroll
      for (int t = 0; t < TOK; ++t) {
        const uint32_t so = (uint32_t)((t < nvalid ? t : nvalid - 1) * v_row);
#pragma unroll
        for (int j = 0; j < NL; ++j) {
          if (FULL || lane_ok) st.v[t][j] = buffer_load16(vrs, past ? 0u : voff[j], so);
          else st.v[t][j] = make_uint4(0u, 0u, 0u, 0u);
        }
      }
      return (!past && phys >= 0) ? nvalid : 0;
    };

    // Folds one step into the online softmax.
    auto consume = [&](const Step<T, TOK>& st, int nvalid) {
      // No implicit FMA contraction: a score and the running max derived from
      // it must be the same rounded value, so the largest score's weight is
      // exactly 2^0 = 1 (explicit fmaf / dot2 calls are unaffected).
#pragma clang fp contract(off)
      float s[TOK];
      float mb = -INFINITY;
#pragma unroll
      for (int t = 0; t < TOK; ++t) {
        const float d = group_sum<LPH>(q.dot(st.k[t])) * a.scale_log2;
        s[t] = t < nvalid ? d : -INFINITY;
        mb = fmaxf(mb, s[t]);
      }
      const float mn = fmaxf(m, mb);
      const float alpha = fast_exp2(m - mn);
      float psum = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] *= alpha;
#pragma unroll
      for (int t = 0; t < TOK; ++t) {
        const float p = fast_exp2(s[t] - mn);
        psum += p;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = fmaf(p, frag_elem<T>(st.v[t], i), acc[i]);
      }
      l = l * alpha + psum;
      m = mn;
    };

    // Two-deep software pipeline: the loads of step s+1 are in flight while
    // step s is folded in.
    Step<T, TOK> A, B;
    int nva = issue(0, A);
    for (int s = 0; s < nsteps; s += 2) {
      const int nvb = issue(s + 1, B);
      __builtin_amdgcn_sched_barrier(0);
      if (nva > 0) consume(A, nva);
      nva = issue(s + 2, A);
      __builtin_amdgcn_sched_barrier(0);
      if (nvb > 0) consume(B, nvb);
    }
  }
}

// Writes a wave's state: the normalised output when the sequence has one
// piece of work, else the partial in workspace slot pidx.
template <typename T>
__device__ __forceinline__ void finish_piece(const DecodeArgs& a, int b, int h, int sub, bool lane_ok,
                                             float m, float l, const float (&acc)[8], int npieces,
                                             size_t pidx) {
  if (!lane_ok) return;
  if (npieces <= 1) {
    store_out<T>(a, b, h, sub, acc, l > 0.f ? 1.f / l : 0.f);
    return;
  }
  float* wa = a.ws_acc + pidx * a.D;
  float4* w0 = reinterpret_cast<float4*>(wa + Layout<T>::elem(sub, a.D, 0));
  float4* w1 = reinterpret_cast<float4*>(wa + Layout<T>::elem(sub, a.D, 4));
  *w0 = make_float4(acc[0], acc[1], acc[2], acc[3]);
  *w1 = make_float4(acc[4], acc[5], acc[6], acc[7]);
  if (sub == 0) a.ws_ml[pidx] = make_float2(m, l);
}

// Partition mode: one wavefront per (HPW heads, partition of part_tokens
// tokens, sequence); partitions past a context exit at once.
template <typename T, int LPH, int TOK, bool FULL>
__global__ void __launch_bounds__(64)
paged_decode_fast(const DecodeArgs a) {
  constexpr int HPW = 64 / LPH;
  const int lane = (int)threadIdx.x;
  const int sub = lane % LPH;
  const int h = (int)blockIdx.x * HPW + lane / LPH;
  const int part = (int)blockIdx.y;
  const int b = (int)blockIdx.z;
  const bool lane_ok = FULL || (h < a.H && sub * 8 < a.D);

  const int ctx = clamp_ctx<T>(a, b);
  const int P = a.part_tokens;
  const int nparts = (ctx + P - 1) / P;
  if (part >= (nparts > 0 ? nparts : 1)) return;  // uniform over the wave

  QFrag<T> q;
  load_query<T>(a, b, h, sub, lane_ok, q);
  uint32_t koff[Layout<T>::kLoads], voff[Layout<T>::kLoads];
  row_offsets<T>(a, h, sub, lane_ok, koff, voff);
  float m = -INFINITY, l = 0.f, acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  const int bpp = P / a.S;  // P is a multiple of S
  if (a.kw != nullptr && ctx == 0 && part == 0) append_row<T, FULL>(a, b, h, sub, lane_ok);
  fold_chunk<T, LPH, TOK, FULL>(a, b, h, lane, lane_ok, q, koff, voff, part * bpp, (part + 1) * bpp, ctx,
                                 m, l, acc);
  finish_piece<T>(a, b, h, sub, lane_ok, m, l, acc, nparts, ((size_t)b * a.H + h) * a.max_parts + part);
}

// Balanced mode. The blocks of all sequences, in sequence order, form one
// list of total = sum_b ceil(ctx_b / S) blocks, cut into P equal segments
// (P = bal_waves, the waves of one head group) of Lw = max(bal_min_blocks,
// ceil(total / P)) blocks, and each segment into claims: contiguous runs of
// the list that one wave streams. A sequence split over several claims gets
// one partial per claim, combined by paged_decode_merge; a sequence inside
// one claim is written directly.
//
// Segment w holds wave w's own claim (about bal_tier1_16ths/16 of it) and R
// ticket claims of a blocks each (R <= bal_tier2, fewer when a would drop
// below bal_min_blocks). A wave streams its own claim, then draws tickets
// from its head group's counter until they run out; ticket t is claim
// 1 + t / P of segment t % P, so the tickets sweep the whole list. The waves
// of a head group are spread over all XCDs (see paged_decode_fast_bal), and
// faster XCDs draw more tickets, so the grid ends together. Measured on
// MI355X, the XCDs of one chip stream at different rates (the slowest about
// 15% behind the fastest at the same load): an equal split leaves the fast
// XCDs idle for the last tenth of the kernel.
//
// The ticket counter is zeroed by wave 0 of its head group when that wave
// starts, and wave 0 draws tickets after its own claim like every other
// wave, so each ticket claim is drawn at least once after the zeroing and no
// claim is skipped. A wave that draws before the zeroing is seen gets a
// stale value: past the last ticket it stops; otherwise it streams a claim
// that is streamed again later. A claim's partials and outputs are a function
// of the claim's index alone, so a second streaming rewrites the same values.
// The workspace needs no initialisation.
//
// Claims are numbered in list order, c = w * (1 + R) + k (k = 0: the own
// claim), and none inside the list is empty, so the pieces of a sequence are
// the consecutive claims from claim_of(cb) to claim_of(ce - 1). Partial slots
// belong to claims, not sequences: a claim holds at most two partials, for
// the sequence it starts in (slot 0: the sequence began at or before the
// claim's first block) and for the one it ends in (slot 1: that sequence
// began inside the claim and runs past its end), since every other sequence
// it touches lies wholly inside it. Slot (h, c, s) is (h * bal_claims + c) *
// 2 + s, bal_claims = P * (1 + bal_tier2), so the workspace holds
// H * bal_claims * 2 partials whatever B and the table width.
struct Claims {
  int total;  // blocks in the list
  int Lw;     // blocks per segment
  int A;      // blocks of a segment's own claim
  int a;      // blocks per ticket claim
  int K;      // claims per segment, 1 + R
};

// Same arithmetic in the attention kernel and the merge (both see the same
// total). With bal_tier2 == 0 every wave streams its whole segment.
__device__ __forceinline__ Claims make_claims(const DecodeArgs& a, int total) {
  Claims c;
  c.total = total;
  const int64_t minb = a.bal_min_blocks;
  int64_t Lw = ((int64_t)total + a.bal_waves - 1) / a.bal_waves;
  if (Lw < minb) Lw = minb;
  c.Lw = (int)Lw;  // <= max(minb, total)
  const int64_t small = Lw * (16 - a.bal_tier1_16ths) / 16;
  int64_t R = small / minb;
  if (R > a.bal_tier2) R = a.bal_tier2;
  c.a = R > 0 ? (int)(small / R) : 0;
  c.K = 1 + (int)R;
  c.A = (int)(Lw - R * c.a);  // >= Lw - small >= 1
  return c;
}
// Claim index of list block pos (0 <= pos < total).
__device__ __forceinline__ int claim_of(const Claims& c, int pos) {
  const int seg = pos / c.Lw;
  const int off = pos - seg * c.Lw;
  return seg * c.K + (off < c.A ? 0 : 1 + (off - c.A) / c.a);
}
// First list block of claim i, and one past its last (empty when equal).
__device__ __forceinline__ int claim_begin(const Claims& c, int i) {
  const int seg = i / c.K, k = i - seg * c.K;
  const int64_t s = (int64_t)seg * c.Lw + (k == 0 ? 0 : c.A + (int64_t)(k - 1) * c.a);
  return (int)min(s, (int64_t)c.total);
}
__device__ __forceinline__ int claim_end(const Claims& c, int i) {
  const int seg = i / c.K, k = i - seg * c.K;
  const int64_t e = (int64_t)seg * c.Lw + c.A + (int64_t)k * c.a;
  return (int)min(e, (int64_t)c.total);
}
__device__ __forceinline__ size_t bal_slot(const DecodeArgs& a, const Claims& c, int h, int i, int cb) {
  return ((size_t)h * a.bal_claims + i) * 2 + (claim_begin(c, i) >= cb ? 0 : 1);
}

// Inclusive prefix sums of ceil(ctx_b / S) into cinc[0 .. B) and the
// clamped context lengths into cctx[0 .. B) (a wave entering a sequence then
// reads its length from LDS instead of waiting on a global load before its
// table loads); returns the total (uniform). One wavefront: lane i covers
// sequences [i*K, i*K + K).
template <typename T>
__device__ __forceinline__ int seq_block_scan(const DecodeArgs& a, int lane, int* cinc, int* cctx) {
  const int K = (a.B + 63) / 64;
  const int b0 = lane * K;
  int sum = 0;
  for (int k = 0; k < K; ++k) {
    const int b = b0 + k;
    if (b < a.B) {
      const int c = clamp_ctx<T>(a, b);
      cctx[b] = c;
      sum += (c + a.S - 1) / a.S;
    }
  }
  int incl = sum;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(incl, d, 64);
    if (lane >= d) incl += y;
  }
  int run = incl - sum;
  for (int k = 0; k < K; ++k) {
    const int b = b0 + k;
    if (b < a.B) {
      run += (cctx[b] + a.S - 1) / a.S;
      cinc[b] = run;
    }
  }
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(__shfl(incl, 63, 64));
}

// Wave-uniform read of cinc[i] (i uniform): kept in a scalar register so the
// buffer descriptors derived from it need no per-lane loops.
__device__ __forceinline__ int uread(const int* cinc, int i) {
  return __builtin_amdgcn_readfirstlane(cinc[i]);
}

template <typename T, int LPH, int TOK, bool FULL>
__global__ void __launch_bounds__(64)
paged_decode_fast_bal(const DecodeArgs a) {
  constexpr int HPW = 64 / LPH;
  __shared__ int cinc[kBalMaxB], cctx[kBalMaxB];
  const int lane = (int)threadIdx.x;
  const int sub = lane % LPH;
  const int ngroups = (a.H + HPW - 1) / HPW;
  // Workgroups go to the 8 XCDs round-robin (workgroup id mod 8). Runs of 8
  // consecutive workgroups share a head group, so each head group's waves,
  // and the tickets they draw, are spread over all XCDs: wave w of head group
  // hg runs on XCD w mod 8. (Any bijection is correct; this one balances.)
  int hg, w;
  {
    const int i = (int)blockIdx.x, P = a.bal_waves;
    const int full = ngroups * 8 * (P / 8);
    if (i < full) {
      const int r = i % (ngroups * 8), q = i / (ngroups * 8);
      hg = r / 8;
      w = q * 8 + r % 8;
    } else {
      hg = (i - full) % ngroups;
      w = 8 * (P / 8) + (i - full) / ngroups;
    }
  }
  const int h = hg * HPW + lane / LPH;
  const bool lane_ok = FULL || (h < a.H && sub * 8 < a.D);

  const int total = seq_block_scan<T>(a, lane, cinc, cctx);
  if (blockIdx.x == 0)  // the merge reads the block list from the workspace
    for (int i = lane; i < a.B; i += 64) a.ws_cinc[i] = cinc[i];
  const Claims cl = make_claims(a, total);
  int* ticket = a.ws_ticket + hg;
  const int n_tickets = a.bal_waves * (cl.K - 1);
  if (n_tickets > 0 && w == 0 && lane == 0)
    __hip_atomic_store(ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  uint32_t koff[Layout<T>::kLoads], voff[Layout<T>::kLoads];
  row_offsets<T>(a, h, sub, lane_ok, koff, voff);

  // Fused append of rows whose sequence has no blocks (no wavefront streams
  // them; padding rows, slot -1, are among them): wave w of each head group
  // checks rows 64 w .. 64 w + 63, one per lane.
  if (a.kw != nullptr) {
    for (int b0 = 64 * w; b0 < a.B; b0 += 64 * a.bal_waves) {
      const int bb = b0 + lane;
      bool write = false;
      if (bb < a.B && cinc[bb] == (bb > 0 ? cinc[bb - 1] : 0)) {
        const int64_t slot = load_index(a.slots, a.sl_i64, (int64_t)bb * a.sl_s);
        write = slot >= 0 && slot < a.N * (int64_t)a.S;
      }
      uint64_t rows = __builtin_amdgcn_ballot_w64(write);
      while (rows) {
        const int i = __builtin_ctzll(rows);
        rows &= rows - 1;
        append_row<T, FULL>(a, b0 + i, h, sub, lane_ok);
      }
    }
  }

  // Streams claim c: one flat loop over chunks of at most kMaxBlocksPerPart
  // blocks of one sequence; the state is written out when the wave leaves a
  // sequence.
  auto run_claim = [&](int c) {
    int pos = claim_begin(cl, c);
    const int end = claim_end(cl, c);
    if (pos >= end) return;  // uniform over the wave
    // The sequence holding list block pos: the first b with cinc[b] > pos.
    int b = 0;
    for (int lo = 0, hi = a.B - 1; lo <= hi;) {
      const int mid = (lo + hi) >> 1;
      if (uread(cinc, mid) > pos) {
        b = mid;
        hi = mid - 1;
      } else {
        lo = mid + 1;
      }
    }
    int cb = 0, ce = 0, ctx = 0;
    QFrag<T> q;
    float m = -INFINITY, l = 0.f, acc[8];
    while (pos < end) {
      if (pos >= ce) {  // entering sequence b
        cb = b > 0 ? uread(cinc, b - 1) : 0;
        ce = uread(cinc, b);
        ctx = uread(cctx, b);
        load_query<T>(a, b, h, sub, lane_ok, q);
        m = -INFINITY;
        l = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0.f;
      }
      const int ch_end = min(min(end, ce), pos + kMaxBlocksPerPart);
      fold_chunk<T, LPH, TOK, FULL>(a, b, h, lane, lane_ok, q, koff, voff, pos - cb, ch_end - cb, ctx, m, l,
                                    acc);
      pos = ch_end;
      if (pos == ce || pos == end) {
        finish_piece<T>(a, b, h, sub, lane_ok, m, l, acc, claim_of(cl, ce - 1) - claim_of(cl, cb) + 1,
                        bal_slot(a, cl, h, c, cb));
        // Next sequence with blocks past pos (cinc[B-1] = total bounds b while pos < end).
        while (pos < end && uread(cinc, b) <= pos) ++b;
      }
    }
  };

  run_claim(w * cl.K);  // this wave's own claim
  while (n_tickets > 0) {  // then ticket claims: claim 1 + t / P of segment t % P
    int t = 0;
    if (lane == 0) t = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    t = __builtin_amdgcn_readlane(t, 0);
    if ((unsigned)t >= (unsigned)n_tickets) break;  // uniform over the wave
    run_claim((t % a.bal_waves) * cl.K + 1 + t / a.bal_waves);
  }
}

// Combines the partials of every (b, h) whose context spans more than one
// piece of work (partition mode: ceil(ctx / part_tokens) partitions;
// balanced mode: the claims its blocks fall in). One wavefront per (sequence,
// HPW heads), the fast kernel's head grouping: in each head row, lane j loads
// the (max, sum) of partial p0 + j while every lane loads its 8 elements of
// all CH partial outputs of the chunk, so a chunk costs one round trip;
// chunks fold online:
//   M' = max(M, max_j m_j), L' = L 2^(M-M') + sum_j l_j 2^(m_j-M'),
//   O' = O 2^(M-M') + sum_j O_j 2^(m_j-M').
// In balanced mode it also writes the zero output of a sequence with no
// blocks, which no attention wave visits.
//
// With MW > 1 wavefronts per workgroup (small grids, where each (sequence,
// head group) has many partials), wavefront w folds chunks w, w + MW, ... and
// wavefront 0 combines the MW states through LDS with the same recurrence.
template <typename T, int LPH, int MW>
__global__ void __launch_bounds__(64 * MW)
paged_decode_merge(const DecodeArgs a) {
  constexpr int HPW = 64 / LPH;
  constexpr int CH = LPH < 16 ? LPH : 16;  // partials per chunk
  const int lane = (int)threadIdx.x & 63;
  const int wv = (int)threadIdx.x >> 6;
  const int sub = lane % LPH;
  const int row = lane / LPH;
  const int b = (int)blockIdx.y;
  const int h = (int)blockIdx.x * HPW + row;
  const int D = a.D;
  const bool head_ok = h < a.H;
  const bool lane_ok = head_ok && sub * 8 < D;
  const int hh = head_ok ? h : 0;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  int nparts, cb = 0, c_first = 0;
  Claims cl{};
  if (a.bal_waves > 0) {
    const int total = a.ws_cinc[a.B - 1];
    cb = b > 0 ? a.ws_cinc[b - 1] : 0;
    const int ce = a.ws_cinc[b];
    if (ce <= cb) {  // no blocks: zeros, as for an empty context
      if (lane_ok && wv == 0) store_out<T>(a, b, h, sub, acc, 0.f);
      return;
    }
    cl = make_claims(a, total);
    c_first = claim_of(cl, cb);
    nparts = claim_of(cl, ce - 1) - c_first + 1;
  } else {
    const int ctx = clamp_ctx<T>(a, b);
    nparts = (ctx + a.part_tokens - 1) / a.part_tokens;
  }
  if (nparts <= 1) return;  // uniform over the wave
  // Workspace slot of partial j of (b, hh).
  auto slot = [&](int j) -> size_t {
    return a.bal_waves > 0 ? bal_slot(a, cl, hh, c_first + j, cb)
                           : ((size_t)b * a.H + hh) * a.max_parts + j;
  };

  float M = -INFINITY, L = 0.f;
  for (int p0 = wv * CH; p0 < nparts; p0 += MW * CH) {
    float2 ml = make_float2(-INFINITY, 0.f);
    if (head_ok && sub < CH && p0 + sub < nparts) ml = a.ws_ml[slot(p0 + sub)];
    float4 x0[CH], x1[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (lane_ok && p0 + j < nparts) {
        const float* wa = a.ws_acc + slot(p0 + j) * D;
        x0[j] = *reinterpret_cast<const float4*>(wa + Layout<T>::elem(sub, D, 0));
        x1[j] = *reinterpret_cast<const float4*>(wa + Layout<T>::elem(sub, D, 4));
      } else {
        x0[j] = x1[j] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    const float Mn = fmaxf(M, group_reduce<LPH, MaxOp>(ml.x));
    const float alpha = (M == Mn) ? 1.f : fast_exp2(M - Mn);
    const float w = (ml.x == -INFINITY) ? 0.f : fast_exp2(ml.x - Mn);
    L = L * alpha + group_sum<LPH>(w * ml.y);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= alpha;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const float wj = __shfl(w, row * LPH + j, 64);  // weight of partial p0 + j
      acc[0] = fmaf(wj, x0[j].x, acc[0]);
      acc[1] = fmaf(wj, x0[j].y, acc[1]);
      acc[2] = fmaf(wj, x0[j].z, acc[2]);
      acc[3] = fmaf(wj, x0[j].w, acc[3]);
      acc[4] = fmaf(wj, x1[j].x, acc[4]);
      acc[5] = fmaf(wj, x1[j].y, acc[5]);
      acc[6] = fmaf(wj, x1[j].z, acc[6]);
      acc[7] = fmaf(wj, x1[j].w, acc[7]);
    }
    M = Mn;
  }
  if constexpr (MW > 1) {
    // Combine the wavefronts' states: M = max_w M_w, L = sum_w L_w 2^(M_w - M),
    // O = sum_w O_w 2^(M_w - M). A wavefront with no chunk has M_w = -inf.
    __shared__ float st_m[MW][64], st_l[MW][64], st_o[MW][8][64];
    st_m[wv][lane] = M;
    st_l[wv][lane] = L;
#pragma unroll
    for (int i = 0; i < 8; ++i) st_o[wv][i][lane] = acc[i];
    __syncthreads();
    if (wv != 0) return;
    M = -INFINITY;
#pragma unroll
    for (int w = 0; w < MW; ++w) M = fmaxf(M, st_m[w][lane]);
    L = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.f;
#pragma unroll
    for (int w = 0; w < MW; ++w) {
      const float mw = st_m[w][lane];
      const float f = mw == -INFINITY ? 0.f : fast_exp2(mw - M);
      L = fmaf(f, st_l[w][lane], L);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = fmaf(f, st_o[w][i][lane], acc[i]);
    }
  }
  if (!lane_ok) return;
  store_out<T>(a, b, h, sub, acc, L > 0.f ? 1.f / L : 0.f);
}

// ----------------------------------------------------------- generic kernel
// One wavefront per (b, h); lane owns d = lane + 64*j. Any strides, any S.
constexpr int kGenericMaxD = 512;

template <typename T>
__global__ void __launch_bounds__(64)
paged_decode_generic(const DecodeArgs a) {
  constexpr int NJ = kGenericMaxD / 64;
  const int lane = (int)threadIdx.x;
  const int h = (int)blockIdx.x;
  const int b = (int)blockIdx.y;
  const int D = a.D;
  const int ctx = clamp_ctx<T>(a, b);

  const T* qrow = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;
  float q[NJ], acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int d = lane + 64 * j;
    q[j] = d < D ? Elem<T>::load(qrow + (int64_t)d * a.q_sd) : 0.f;
    acc[j] = 0.f;
  }
  const T* kh = reinterpret_cast<const T*>(a.k) + (int64_t)h * a.k_sh;
  const T* vh = reinterpret_cast<const T*>(a.v) + (int64_t)h * a.v_sh;
  const int64_t bt_row = (int64_t)b * a.bt_sb;
  float m = -INFINITY, l = 0.f;
  int blk = 0, off = 0;
  int64_t phys = 0;
  for (int t = 0; t < ctx; ++t) {
#pragma clang fp contract(off)
    if (off == 0) phys = load_index(a.bt, a.bt_i64, bt_row + (int64_t)blk * a.bt_sm);
    if (phys >= 0 && phys < a.N) {
      const T* kt = kh + phys * a.k_sn + (int64_t)off * a.k_ss;
      const T* vt = vh + phys * a.v_sn + (int64_t)off * a.v_ss;
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int d = lane + 64 * j;
        if (d < D) part = fmaf(q[j], Elem<T>::load(kt + (int64_t)d * a.k_sd), part);
      }
      const float s = wave_sum(part) * a.scale_log2;
      const float mn = fmaxf(m, s);
      const float alpha = fast_exp2(m - mn);
      const float p = fast_exp2(s - mn);
      l = l * alpha + p;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int d = lane + 64 * j;
        const float v = d < D ? Elem<T>::load(vt + (int64_t)d * a.v_sd) : 0.f;
        acc[j] = fmaf(p, v, acc[j] * alpha);
      }
      m = mn;
    }
    if (++off == a.S) {
      off = 0;
      ++blk;
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  T* orow = reinterpret_cast<T*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int d = lane + 64 * j;
    if (d < D) Elem<T>::store(orow + (int64_t)d * a.o_sd, acc[j] * inv);
  }
}

// ---------------------------------------------------------------- launchers
static hipError_t launch(const void* fn, dim3 grid, dim3 block, const DecodeArgs& a,
                         hipStream_t stream) {
  void* args[] = {const_cast<DecodeArgs*>(&a)};
  return hipLaunchKernel(fn, grid, block, args, 0, stream);
}

template <typename T, int LPH>
static hipError_t launch_merge(const DecodeArgs& a, hipStream_t stream) {
  constexpr int HPW = 64 / LPH;
  const dim3 mgrid((unsigned)((a.H + HPW - 1) / HPW), (unsigned)a.B);
  switch (a.merge_waves) {
    case 8: return launch(reinterpret_cast<const void*>(&paged_decode_merge<T, LPH, 8>), mgrid, dim3(512), a, stream);
    case 4: return launch(reinterpret_cast<const void*>(&paged_decode_merge<T, LPH, 4>), mgrid, dim3(256), a, stream);
    case 2: return launch(reinterpret_cast<const void*>(&paged_decode_merge<T, LPH, 2>), mgrid, dim3(128), a, stream);
    default: return launch(reinterpret_cast<const void*>(&paged_decode_merge<T, LPH, 1>), mgrid, dim3(64), a, stream);
  }
}

template <typename T, int LPH, int TOK>
static hipError_t launch_fast_lph_tok(const DecodeArgs& a, bool full, hipStream_t stream) {
  constexpr int HPW = 64 / LPH;
  const unsigned ngroups = (unsigned)((a.H + HPW - 1) / HPW);
  hipError_t e;
  if (a.bal_waves > 0) {
    const void* fn = full ? reinterpret_cast<const void*>(&paged_decode_fast_bal<T, LPH, TOK, true>)
                          : reinterpret_cast<const void*>(&paged_decode_fast_bal<T, LPH, TOK, false>);
    e = launch(fn, dim3(ngroups * (unsigned)a.bal_waves), dim3(64), a, stream);
  } else {
    const void* fn = full ? reinterpret_cast<const void*>(&paged_decode_fast<T, LPH, TOK, true>)
                          : reinterpret_cast<const void*>(&paged_decode_fast<T, LPH, TOK, false>);
    e = launch(fn, dim3(ngroups, (unsigned)a.max_parts, (unsigned)a.B), dim3(64), a, stream);
  }
  if (e != hipSuccess || (a.bal_waves <= 0 && a.max_parts <= 1)) return e;
  return launch_merge<T, LPH>(a, stream);
}

template <typename T, int LPH>
static hipError_t launch_fast_lph(const DecodeArgs& a, const DecodePlan& p, hipStream_t stream) {
  if constexpr (sizeof(T) == 2) {
    if (p.tokens_per_step == 16) return launch_fast_lph_tok<T, LPH, 16>(a, p.full_lanes, stream);
    if (p.tokens_per_step == 8) return launch_fast_lph_tok<T, LPH, 8>(a, p.full_lanes, stream);
  } else {
    if (p.tokens_per_step == 8) return launch_fast_lph_tok<T, LPH, 8>(a, p.full_lanes, stream);
    if (p.tokens_per_step == 4) return launch_fast_lph_tok<T, LPH, 4>(a, p.full_lanes, stream);
  }
  return hipErrorInvalidValue;
}

template <typename T>
static hipError_t launch_fast(const DecodeArgs& a, const DecodePlan& p, hipStream_t stream) {
  switch (p.lanes_per_head) {
    case 4: return launch_fast_lph<T, 4>(a, p, stream);
    case 8: return launch_fast_lph<T, 8>(a, p, stream);
    case 16: return launch_fast_lph<T, 16>(a, p, stream);
    case 32: return launch_fast_lph<T, 32>(a, p, stream);
    default: return hipErrorInvalidValue;
  }
}

template <typename T>
static hipError_t launch_generic(const DecodeArgs& a, hipStream_t stream) {
  return launch(reinterpret_cast<const void*>(&paged_decode_generic<T>),
                dim3((unsigned)a.H, (unsigned)a.B), dim3(64), a, stream);
}

template <typename T>
static hipError_t launch_merge_lph(const DecodeArgs& a, int lanes_per_head, hipStream_t stream) {
  switch (lanes_per_head) {
    case 4: return launch_merge<T, 4>(a, stream);
    case 8: return launch_merge<T, 8>(a, stream);
    case 16: return launch_merge<T, 16>(a, stream);
    case 32: return launch_merge<T, 32>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_paged_merge(const DecodeArgs& a, int dtype, int lanes_per_head, hipStream_t stream) {
  if (dtype == MGI_BF16) return launch_merge_lph<bf16_t>(a, lanes_per_head, stream);
  if (dtype == MGI_F16) return launch_merge_lph<f16_t>(a, lanes_per_head, stream);
  if (dtype == MGI_F32) return launch_merge_lph<float>(a, lanes_per_head, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_paged_decode(const DecodeArgs& a, int dtype, const DecodePlan& plan,
                               hipStream_t stream) {
  if (plan.path == DecodePath::kFast) {
    if (dtype == MGI_BF16) return launch_fast<bf16_t>(a, plan, stream);
    if (dtype == MGI_F32) return launch_fast<float>(a, plan, stream);
    if (dtype == MGI_F16) return launch_fast<f16_t>(a, plan, stream);
    return hipErrorInvalidValue;
  }
  if (dtype == MGI_BF16) return launch_generic<bf16_t>(a, stream);
  if (dtype == MGI_F32) return launch_generic<float>(a, stream);
  if (dtype == MGI_F16) return launch_generic<f16_t>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace mgi
