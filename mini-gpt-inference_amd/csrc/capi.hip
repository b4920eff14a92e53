// capi.hip -- extern "C" entry points of libminivllm_hip.so (declared in
// include/minivllm_hip.h): argument validation, path selection, workspace
// layout and launch. Validation mirrors the host checks of
// paged_attention_batch_triton_v0 (minivllm/triton_paged_decode.py:109-144);
// nothing here reads device memory or synchronises the stream.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <mutex>
#include <string>

#include "mgi_internal.h"
#include "minivllm_hip.h"

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

bool valid_dtype(int d) { return d == MGI_F32 || d == MGI_BF16 || d == MGI_F16; }
bool valid_itype(int t) { return t == MGI_I32 || t == MGI_I64; }
int64_t dtype_bytes(int d) { return d == MGI_F32 ? 4 : 2; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool mult16(int64_t elems, int64_t eb) { return (elems * eb) % 16 == 0; }

bool nonneg(const int64_t* s, int n) {
  for (int i = 0; i < n; ++i)
    if (s[i] < 0) return false;
  return true;
}

constexpr int64_t kMaxGridYZ = 65535;
constexpr int64_t kWorkspaceAlign = 256;

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Blocks one partition of the fast kernel may span (its block-table entries
// live in two VGPRs of the wavefront).
constexpr int64_t kMaxBlocksPerPart = 128;

// Compute units of the current device (256 on MI355X; 256 when no device is
// visible, e.g. for host-only size queries).
int device_cus() {
  static std::atomic<int> cached[64];  // 0 = not queried yet (zero-initialised)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (!n) {
    int q = 0;
    n = (hipDeviceGetAttribute(&q, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && q > 0) ? q : 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Partition size in tokens: a multiple of S, at most kMaxBlocksPerPart blocks
// and at most the table's M*S. Automatic choice: the smallest power of two
// >= 256 for which the grid, sized for contexts filling the table, holds
// about four wavefronts per SIMD of the chip (4 heads per wavefront at
// head_dim 128). Measured on MI355X: ragged 512-4096 contexts at B=64 and
// 32k-128k contexts at B=8 both sit within ~1% of their best split there.
int64_t split_tokens_for(int64_t B, int64_t H, int64_t D, int64_t S, int64_t M,
                         int64_t requested) {
  const int64_t max_ctx = M * S;
  int64_t P = requested;
  if (P <= 0) {
    const int64_t lph = D <= 32 ? 4 : D <= 64 ? 8 : D <= 128 ? 16 : 32;
    const int64_t waves_per_part = B * ((H + 64 / lph - 1) / (64 / lph));
    const int64_t target = 4 * 4 * (int64_t)device_cus();  // 4 SIMDs per CU
    P = 256;
    while (P < max_ctx && waves_per_part * ((max_ctx + P - 1) / P) > target) P *= 2;
  }
  P = std::min(round_up(P, S), kMaxBlocksPerPart * S);
  return std::min(P, max_ctx);
}

// Balanced split of the fast kernel (paged_decode_fast_bal): every wave of a
// head group streams the same number of blocks of the concatenated block
// list of all sequences. Used when the partition split would cut some
// contexts (more than one partition per table) and the caller left the split
// to the library. The waves of all head groups together number three per
// CU, so all of them are resident at once (the fast kernel's registers allow
// one per SIMD) and finish together, each taking at least kBalMinTokens
// tokens. Measured on MI355X (B=64 ragged, B=256, B=8 long contexts; bf16 and
// f32): 2-3 waves per CU are best and within noise of each other; 4 per CU is
// 1-2% slower, and 5-6 per CU (a partial second round) up to 10% slower. A
// floor of 64 tokens per wave halves small calls against 256 (B=8 x 256
// tokens, 16 heads: 16.9 against 34.6 us) and leaves large ones unchanged;
// 16 and 32 are no better. MINIVLLM_HIP_DECODE_BALANCED=0 turns the mode off,
// MINIVLLM_HIP_BAL_WAVES sets the total wave count and
// MINIVLLM_HIP_BAL_MIN_TOKENS the floor (tuning).
constexpr int64_t kBalMinTokens = 64;

int env_int(const char* name, int dflt) {
  const char* e = std::getenv(name);
  return e ? std::atoi(e) : dflt;
}

// Balanced mode's ticket claims (see paged_decode_fast_bal): each wave's own
// claim covers kBalTier1Sixteenths/16 of its segment and the rest is cut into
// up to kBalTier2PerWave claims taken by ticket. Measured on MI355X against
// no ticket claims (16/16): +1.5% at bf16 B=64 x 512-4096, +3% in f32, +1.6%
// at B=256 x 128-2048, +2.3% at B=8 x 32k-128k, +1.2% at a fixed 1024
// context, equal at 512; (14, 3) was best or tied among 12-15 sixteenths and
// 3-6 claims. MINIVLLM_HIP_BAL_TIER1 (sixteenths, 1-16) and
// MINIVLLM_HIP_BAL_TIER2 (claims per segment, 0 turns them off) override
// the choice (tuning; read on every call).
constexpr int kBalTier1Sixteenths = 14;
constexpr int kBalTier2PerWave = 3;

struct SplitPlan {
  int64_t P;             // partition mode: tokens per partition
  int64_t max_parts;     // partition mode: partials per (sequence, head)
  int bal_waves;         // > 0: balanced mode, waves per head group
  int bal_min_blocks;    // balanced mode: least blocks per claim
  int bal_tier1_16ths;   // balanced mode: share of the list in the waves' own claims
  int bal_tier2;         // balanced mode: ticket claims per wave's segment (at most)
  int64_t bal_groups;    // balanced mode: head groups (one ticket counter each)
  int64_t n_partials;    // partial slots in the workspace
};

SplitPlan split_plan(int64_t B, int64_t H, int64_t D, int64_t S, int64_t M, int64_t requested) {
  static const int balanced = env_int("MINIVLLM_HIP_DECODE_BALANCED", 1);
  static const int waves = env_int("MINIVLLM_HIP_BAL_WAVES", 0);
  static const int64_t min_tokens = std::max(1, env_int("MINIVLLM_HIP_BAL_MIN_TOKENS", (int)kBalMinTokens));
  SplitPlan sp{};
  sp.P = split_tokens_for(B, H, D, S, M, requested);
  sp.max_parts = (M * S + sp.P - 1) / sp.P;
  if (balanced && requested <= 0 && sp.max_parts > 1 && B <= mgi::kBalMaxB &&
      B * M < (int64_t(1) << 31)) {
    const int64_t lph = D <= 32 ? 4 : D <= 64 ? 8 : D <= 128 ? 16 : 32;
    const int64_t groups = (H + 64 / lph - 1) / (64 / lph);
    const int64_t target = waves > 0 ? waves : 3 * (int64_t)device_cus();
    sp.bal_waves = (int)std::max<int64_t>(1, target / groups);
    sp.bal_min_blocks = (int)((min_tokens + S - 1) / S);
    sp.bal_tier1_16ths = std::min(16, std::max(1, env_int("MINIVLLM_HIP_BAL_TIER1", kBalTier1Sixteenths)));
    sp.bal_tier2 = std::min(64, std::max(0, env_int("MINIVLLM_HIP_BAL_TIER2", kBalTier2PerWave)));
    sp.bal_groups = groups;
    // two slots per (head, claim); 1 + bal_tier2 claims per wave's segment
    sp.n_partials = H * (int64_t)sp.bal_waves * (1 + sp.bal_tier2) * 2;
  } else if (sp.max_parts > 1) {
    sp.n_partials = B * H * sp.max_parts;
  }
  return sp;
}

struct WorkspaceLayout {
  size_t acc_bytes, ml_offset, cinc_offset, ticket_offset, total;
};

// [acc: n_partials*D f32 | ml: n_partials float2 | cinc: B int32 | ticket:
// one int32 per head group (the last two in balanced mode only)], acc, ml
// and cinc 256-byte aligned. Partition mode holds B*H*max_parts partials;
// balanced mode 2 per (head, claim), whatever B and M. Nothing in it needs
// initialising.
WorkspaceLayout workspace_layout(int64_t B, int64_t D, const SplitPlan& sp) {
  WorkspaceLayout w{};
  if (sp.n_partials == 0) return w;
  const int64_t n = sp.n_partials;
  w.acc_bytes = (size_t)(n * D * 4);
  w.ml_offset = (size_t)round_up((int64_t)w.acc_bytes, kWorkspaceAlign);
  w.cinc_offset = (size_t)round_up((int64_t)w.ml_offset + n * 8, kWorkspaceAlign);
  w.ticket_offset = w.cinc_offset + (size_t)(B * 4);
  w.total = sp.bal_waves > 0 ? w.ticket_offset + (size_t)(sp.bal_groups * 4)
                             : w.ml_offset + (size_t)(n * 8);
  return w;
}

// Tokens loaded per pipeline stage of the fast kernel: 16 for bf16 and f16
// and 8 for f32 (32 KiB of K+V per stage and wavefront at head_dim 128; two
// stages in flight), or the largest S allows. Measured on MI355X this beats
// smaller stages at higher occupancy on large calls. Small 2-byte calls,
// whose table bound B*M*S*H*D*2 elements is at most kSmallCallKvBytes, take 8:
// each wave's stream is short there and smaller stages end it with less
// imbalance (B=64 x U[512, 4096], 4 heads: 62.3 -> 60.2 us; 8 heads: 112.3
// -> 109.7 us; B=16 x 32 heads: 102.7 -> 100.4 us; 16 heads, a 2.1 GB bound:
// 201.5 -> 206.8 us the other way). MINIVLLM_HIP_TOKENS_PER_STEP (8 or 16
// for the 2-byte types, 4 or 8 for f32) overrides the choice when S allows it
// (tuning).
constexpr double kSmallCallKvBytes = 1.5e9;
int tokens_per_step_override() {
  static const int v = [] {
    const char* e = std::getenv("MINIVLLM_HIP_TOKENS_PER_STEP");
    return e ? std::atoi(e) : 0;
  }();
  return v;
}

int next_pow2_at_least4(int64_t x) {
  int p = 4;
  while (p < x) p *= 2;
  return p;
}

// Rows of a chunk at contexts start+1 .. start+T whose keys span several
// partitions of pk keys, counted once per partition they span.
int64_t split_partials(int64_t start, int64_t T, int64_t pk) {
  int64_t n = 0;
  for (int64_t j = 2; (j - 1) * pk < start + T; ++j) {
    const int64_t lo = std::max(start + 1, (j - 1) * pk + 1), hi = std::min(start + T, j * pk);
    if (hi >= lo) n += (hi - lo + 1) * j;
  }
  return n;
}

// Paged prefill key split: keys per partition, or 0 for none. A chunk whose
// workgroups (one per 64-row query tile and head, 32 rows for chunks of at
// most 32) are fewer than two per CU leaves CUs idle and waits on its last
// query tile, which folds every key tile of the prefix. Splitting each query
// tile's keys into partitions of k tiles, k about the total key tiles over
// two per CU (at least 2), spreads that work; the partials are combined by
// paged_decode_merge. The split is taken when a cost model fitted on MI355X
// (bf16, head_dim 128, 8-32 heads, chunks of 64-2048 rows after prefixes of
// 0-16k tokens) says it pays: a lone workgroup takes ~1.5 us per 64-key
// tile (scaled with head_dim), and the split adds ~8 us (merge launch, tail)
// plus its fp32 partials written and read back at ~5 TB/s. It pays after
// long prefixes (a 256-row chunk after 3000 tokens, 32 heads: 80 -> 41 us)
// and not for chunks whose causal triangle is most of the work (a 512-row
// chunk at position 0: 18 -> 26 us split), so it needs a prefix at least as
// long as the chunk: the model alone would split a 1024-row first chunk of
// 16 heads, measured 28.9 -> 34.1 us (two workgroups per CU slow each tile
// and the diagonal tiles take the masking path). 2-byte types with head_dim
// a multiple of 8 only (the merge's lane layout).
// MINIVLLM_HIP_PREFILL_SPLIT_KEYS = -1 turns it off; > 0 forces that many
// keys per partition, rounded up to 64, without the cost model (tuning and
// tests; read on every call).
int64_t prefill_split_keys(int64_t start, int64_t T, int64_t H, int64_t D, int dtype) {
  const int forced = env_int("MINIVLLM_HIP_PREFILL_SPLIT_KEYS", 0);
  if (forced < 0 || dtype == MGI_F32 || D % 8 != 0 || mgi::prefill_head_dim_bucket(1, (int)D) == 0 ||
      T <= 0 || T > kMaxGridYZ)
    return 0;
  const int64_t QB = T <= 32 ? 32 : 64;
  const int64_t nq = (T + QB - 1) / QB;
  int64_t total = 0, longest = 0;
  for (int64_t qt = 0; qt < nq; ++qt) {
    const int64_t tiles = (start + std::min(T, (qt + 1) * QB) + 63) / 64;
    total += tiles;
    longest = std::max(longest, tiles);
  }
  if (forced > 0) {
    const int64_t pk = round_up(forced, 64);
    return pk < longest * 64 && (start + T + pk - 1) / pk <= kMaxGridYZ ? pk : 0;  // partitions: grid y
  }
  const int64_t slots = 2 * (int64_t)device_cus();
  if (nq * H >= slots || start < T) return 0;
  const int64_t k = std::max<int64_t>(2, (total * H + slots - 1) / slots);
  if (k >= longest) return 0;
  const double tile_us = 1.5 * (double)std::max<int64_t>(D, 64) / 128.0;
  const double partial_bytes = (double)split_partials(start, T, 64 * k) * (double)H * (double)(4 * D + 8);
  const double split_us = (double)k * tile_us + 8.0 + 2.0 * partial_bytes / 5.0e6;
  return split_us < (double)longest * tile_us && (start + T + 64 * k - 1) / (64 * k) <= kMaxGridYZ ? 64 * k : 0;
}

struct PrefillWorkspace {
  int64_t part_keys, max_parts;
  size_t ml_offset, total;
};

// [acc: T*H*max_parts*D f32 | ml: T*H*max_parts float2], 256-byte aligned.
PrefillWorkspace prefill_workspace(int64_t start, int64_t T, int64_t H, int64_t D, int dtype) {
  PrefillWorkspace w{};
  w.part_keys = prefill_split_keys(start, T, H, D, dtype);
  if (w.part_keys == 0) return w;
  w.max_parts = (start + T + w.part_keys - 1) / w.part_keys;
  const int64_t n = T * H * w.max_parts;
  w.ml_offset = (size_t)round_up(n * D * 4, kWorkspaceAlign);
  w.total = w.ml_offset + (size_t)(n * 8);
  return w;
}

// Scratch of mgi_paged_decode_noalloc: the split workspace of callers that
// cannot allocate. One copy per device, resident for the life of the process.
// In host code `scratch` names a host-side stand-in; its device address comes
// from hipGetSymbolAddress, per device (each holds its own copy), and only
// that address is handed to kernels. Nothing in the workspace needs to start
// at zero (the kernels write every partial before it is read and zero the
// ticket counters themselves), so the array is used as found.
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device `stream` belongs to (the current
// device for the null stream), resolved on the first call for that device
// with it current.
int scratch_for_stream(hipStream_t stream, void** ptr) {
  int dev = -1;
  if (stream) {
    if (hipStreamGetDevice(stream, &dev) != hipSuccess) return fail(MGI_EINVAL, "invalid stream");
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return fail(MGI_ELAUNCH, "no current HIP device");
  }
  if (dev < 0 || dev >= kMaxDevices) return fail(MGI_EUNSUPPORTED, "device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return fail(MGI_ELAUNCH, "no current HIP device");
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return fail(MGI_ELAUNCH, "cannot select the stream's device");
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p)
      return fail(MGI_ELAUNCH, std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return MGI_OK;
}

}  // namespace

extern "C" {

const char* mgi_last_error(void) { return g_err.c_str(); }

int mgi_abi_version(void) { return 104; }

int64_t mgi_paged_decode_split_tokens(int64_t B, int64_t H, int64_t D, int64_t S, int64_t M,
                                      int64_t split_tokens) {
  if (B <= 0 || H <= 0 || D <= 0 || S <= 0 || M <= 0) return 0;
  return split_tokens_for(B, H, D, S, M, split_tokens);
}

int64_t mgi_paged_decode_balanced_waves(int64_t B, int64_t H, int64_t D, int64_t S, int64_t M,
                                        int64_t split_tokens) {
  if (B <= 0 || H <= 0 || D <= 0 || S <= 0 || M <= 0) return 0;
  return split_plan(B, H, D, S, M, split_tokens).bal_waves;
}

size_t mgi_paged_prefill_workspace_bytes(int64_t start_pos, int64_t T, int64_t H, int64_t D, int dtype) {
  if (start_pos < 0 || T <= 0 || H <= 0 || D <= 0 || !valid_dtype(dtype)) return 0;
  return prefill_workspace(start_pos, T, H, D, dtype).total;
}

size_t mgi_paged_decode_workspace_bytes(int64_t B, int64_t H, int64_t D, int64_t S, int64_t M,
                                        int64_t split_tokens) {
  if (B <= 0 || H <= 0 || D <= 0 || S <= 0 || M <= 0) return 0;
  return workspace_layout(B, D, split_plan(B, H, D, S, M, split_tokens)).total;
}

}  // extern "C"

namespace {

// The new rows of a KV append: mgi_kv_append's arguments, and those of
// mgi_paged_decode_append's append.
struct AppendSpec {
  void* k_pool;
  void* v_pool;
  const void* k_new;
  const void* v_new;
  const int64_t* kn_strides;  // [3]
  const int64_t* vn_strides;  // [3]
  int new_dtype;
  const void* slots;
  int64_t slot_stride;
  int slot_itype;
};

// Checks of the new rows (the pool's are the caller's).
int check_append(const AppendSpec& ap, int pool_dtype, int64_t T) {
  if (!ap.k_new || !ap.v_new || !ap.slots) return fail(MGI_EINVAL, "null tensor pointer");
  if (!ap.kn_strides || !ap.vn_strides) return fail(MGI_EINVAL, "null stride array");
  if (!valid_dtype(ap.new_dtype)) return fail(MGI_EINVAL, "unknown dtype code");
  if (!valid_itype(ap.slot_itype)) return fail(MGI_EINVAL, "slot_mapping must be int32 or int64");
  if (!nonneg(ap.kn_strides, 3) || !nonneg(ap.vn_strides, 3) || ap.slot_stride < 0)
    return fail(MGI_EINVAL, "strides must be non-negative");
  if (T > (int64_t(1) << 31) - 1) return fail(MGI_EUNSUPPORTED, "too many rows");
  if (pool_dtype != ap.new_dtype && pool_dtype != MGI_F32 && ap.new_dtype != MGI_F32)
    return fail(MGI_EUNSUPPORTED, "only same-dtype copies and conversions to/from f32");
  return MGI_OK;
}

// Launches the append kernel for T checked rows.
int launch_append(const AppendSpec& ap, const int64_t* k_pool_strides, const int64_t* v_pool_strides,
                  int pool_dtype, int64_t T, int64_t H, int64_t D, int64_t S, int64_t N,
                  int64_t layer_idx, hipStream_t stream) {
  using namespace mgi;
  const int new_dtype = ap.new_dtype;
  const int64_t* k_new_strides = ap.kn_strides;
  const int64_t* v_new_strides = ap.vn_strides;
  const int64_t peb = dtype_bytes(pool_dtype), neb = dtype_bytes(new_dtype);
  char* kbase = static_cast<char*>(ap.k_pool) + layer_idx * k_pool_strides[0] * peb;
  char* vbase = static_cast<char*>(ap.v_pool) + layer_idx * v_pool_strides[0] * peb;

  AppendArgs a{};
  a.kp = kbase;
  a.vp = vbase;
  a.k_sn = k_pool_strides[1];
  a.k_ss = k_pool_strides[2];
  a.k_sh = k_pool_strides[3];
  a.k_sd = k_pool_strides[4];
  a.v_sn = v_pool_strides[1];
  a.v_ss = v_pool_strides[2];
  a.v_sh = v_pool_strides[3];
  a.v_sd = v_pool_strides[4];
  a.kn = ap.k_new;
  a.vn = ap.v_new;
  a.kn_st = k_new_strides[0];
  a.kn_sh = k_new_strides[1];
  a.kn_sd = k_new_strides[2];
  a.vn_st = v_new_strides[0];
  a.vn_sh = v_new_strides[1];
  a.vn_sd = v_new_strides[2];
  a.slots = ap.slots;
  a.sl_s = ap.slot_stride;
  a.sl_i64 = ap.slot_itype == MGI_I64;
  a.T = (int)T;
  a.H = (int)H;
  a.D = (int)D;
  a.S = (int)S;
  a.N = N;

  const bool rows_contig = k_pool_strides[4] == 1 && k_pool_strides[3] == D &&
                           v_pool_strides[4] == 1 && v_pool_strides[3] == D &&
                           k_new_strides[2] == 1 && k_new_strides[1] == D &&
                           v_new_strides[2] == 1 && v_new_strides[1] == D;
  const bool vector_path = pool_dtype == new_dtype && rows_contig && mult16(H * D, peb) &&
                           aligned16(kbase) && aligned16(vbase) && aligned16(ap.k_new) &&
                           aligned16(ap.v_new) && mult16(k_pool_strides[1], peb) &&
                           mult16(k_pool_strides[2], peb) && mult16(v_pool_strides[1], peb) &&
                           mult16(v_pool_strides[2], peb) && mult16(k_new_strides[0], neb) &&
                           mult16(v_new_strides[0], neb);

  const hipError_t e = launch_kv_append(a, pool_dtype, new_dtype, vector_path, stream);
  if (e != hipSuccess) return fail(MGI_ELAUNCH, std::string("launch failed: ") + hipGetErrorString(e));
  return MGI_OK;
}

// The body of mgi_paged_decode, mgi_paged_decode_noalloc and
// mgi_paged_decode_append. With `use_scratch` the workspace is the device's
// allocation-free scratch (resolved here once the call is known to need it,
// after every check has passed); otherwise it is the caller's `workspace`.
// With `ap`, B new rows are appended first: inside the decode launch on the
// fast path when the rows share the pool's dtype and are 16-byte aligned with
// a contiguous head dim, else by the append kernel launched before it.
int paged_decode_impl(void* out, const int64_t* out_strides, const void* q,
                      const int64_t* q_strides, const void* k_pool, const void* v_pool,
                      const int64_t* k_pool_strides, const int64_t* v_pool_strides, int dtype,
                      const void* block_tables, const int64_t* bt_strides, int bt_itype,
                      const void* context_lens, int64_t cl_stride, int cl_itype, int64_t B,
                      int64_t H, int64_t D, int64_t S, int64_t N, int64_t M, int64_t L,
                      int64_t layer_idx, float scale, int64_t split_tokens, void* workspace,
                      size_t workspace_bytes, bool use_scratch, const AppendSpec* ap, void* stream) {
  using namespace mgi;
  g_err.clear();
  if (!out || !q || !k_pool || !v_pool || !block_tables || !context_lens)
    return fail(MGI_EINVAL, "null tensor pointer");
  if (!out_strides || !q_strides || !k_pool_strides || !v_pool_strides || !bt_strides)
    return fail(MGI_EINVAL, "null stride array");
  if (B <= 0 || H <= 0 || D <= 0) return fail(MGI_EINVAL, "q dimensions must be nonzero");
  if (S <= 0 || N <= 0 || L <= 0) return fail(MGI_EINVAL, "pool dimensions must be nonzero");
  if (M < 1) return fail(MGI_EINVAL, "block_tables need at least one block column");
  if (layer_idx < 0 || layer_idx >= L) return fail(MGI_EINVAL, "layer_idx outside KV pool");
  if (!valid_dtype(dtype)) return fail(MGI_EINVAL, "unknown dtype code");
  if (!valid_itype(bt_itype) || !valid_itype(cl_itype))
    return fail(MGI_EINVAL, "index arrays must be int32 or int64");
  if (!std::isfinite(scale)) return fail(MGI_EINVAL, "scale must be finite");
  if (!nonneg(out_strides, 3) || !nonneg(q_strides, 3) || !nonneg(k_pool_strides, 5) ||
      !nonneg(v_pool_strides, 5) || !nonneg(bt_strides, 2) || cl_stride < 0)
    return fail(MGI_EINVAL, "strides must be non-negative");
  if (B > kMaxGridYZ) return fail(MGI_EUNSUPPORTED, "batch larger than 65535");
  if (M > kMaxGridYZ * kMaxBlocksPerPart)
    return fail(MGI_EUNSUPPORTED, "block table wider than 65535 partitions");
  if (M * S >= (int64_t(1) << 31)) return fail(MGI_EUNSUPPORTED, "M*S must be < 2^31");
  if (D > 512) return fail(MGI_EUNSUPPORTED, "head_dim larger than 512");
  if (ap) {
    const int rc = check_append(*ap, dtype, B);
    if (rc != MGI_OK) return rc;
  }

  const int64_t eb = dtype_bytes(dtype);
  const char* kbase = static_cast<const char*>(k_pool) + layer_idx * k_pool_strides[0] * eb;
  const char* vbase = static_cast<const char*>(v_pool) + layer_idx * v_pool_strides[0] * eb;

  const SplitPlan sp = split_plan(B, H, D, S, M, split_tokens);
  const WorkspaceLayout ws = workspace_layout(B, D, sp);

  // Path selection: the fast kernel needs unit d-stride, 16-byte aligned head
  // rows, head_dim a multiple of 8 up to 256 and S a multiple of its step.
  DecodePlan plan{};
  plan.path = DecodePath::kGeneric;
  const int64_t row_span = ((H - 1) * std::max(k_pool_strides[3], v_pool_strides[3]) + D) * eb;
  if (D % 8 == 0 && D <= 256 &&
      k_pool_strides[4] == 1 && v_pool_strides[4] == 1 && aligned16(kbase) &&
      aligned16(vbase) && mult16(k_pool_strides[1], eb) && mult16(k_pool_strides[2], eb) &&
      mult16(k_pool_strides[3], eb) && mult16(v_pool_strides[1], eb) &&
      mult16(v_pool_strides[2], eb) && mult16(v_pool_strides[3], eb) &&
      row_span < (int64_t(1) << 31) &&
      std::max(k_pool_strides[2], v_pool_strides[2]) * eb * S < (int64_t(1) << 31)) {
    int tok = 0;
    const int want = tokens_per_step_override();
    const bool two_byte = dtype != MGI_F32;
    const double kv_bound = (double)B * (double)M * (double)S * (double)H * (double)D * (double)eb * 2.0;
    const int def = two_byte ? (kv_bound <= kSmallCallKvBytes ? 8 : 16) : 8;
    for (int t : {want, def, 8, 4}) {
      if (t > 0 && ((two_byte && (t == 8 || t == 16)) || (!two_byte && (t == 4 || t == 8))) &&
          S % t == 0) {
        tok = t;
        break;
      }
    }
    if (tok) {
      plan.path = DecodePath::kFast;
      plan.tokens_per_step = tok;
      plan.lanes_per_head = next_pow2_at_least4(D / 8);
      plan.full_lanes = (D == 8 * plan.lanes_per_head) && (H % (64 / plan.lanes_per_head) == 0);
    }
  }

  // Partition mode launches one grid row per partition.
  if (plan.path == DecodePath::kFast && sp.bal_waves == 0 && sp.max_parts > kMaxGridYZ)
    return fail(MGI_EUNSUPPORTED, "more than 65535 partitions per context (split_tokens too small for the table)");

  DecodeArgs a{};
  a.out = out;
  a.o_sb = out_strides[0];
  a.o_sh = out_strides[1];
  a.o_sd = out_strides[2];
  a.q = q;
  a.q_sb = q_strides[0];
  a.q_sh = q_strides[1];
  a.q_sd = q_strides[2];
  a.k = kbase;
  a.v = vbase;
  a.k_sn = k_pool_strides[1];
  a.k_ss = k_pool_strides[2];
  a.k_sh = k_pool_strides[3];
  a.k_sd = k_pool_strides[4];
  a.v_sn = v_pool_strides[1];
  a.v_ss = v_pool_strides[2];
  a.v_sh = v_pool_strides[3];
  a.v_sd = v_pool_strides[4];
  a.bt = block_tables;
  a.bt_sb = bt_strides[0];
  a.bt_sm = bt_strides[1];
  a.cl = context_lens;
  a.cl_s = cl_stride;
  a.bt_i64 = bt_itype == MGI_I64;
  a.cl_i64 = cl_itype == MGI_I64;
  a.B = (int)B;
  a.H = (int)H;
  a.D = (int)D;
  a.S = (int)S;
  a.M = (int)M;
  a.N = N;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.part_tokens = (int)sp.P;
  a.max_parts = plan.path == DecodePath::kFast ? (int)sp.max_parts : 1;
  if (plan.path == DecodePath::kFast && sp.n_partials > 0) {
    if (use_scratch) {
      if (ws.total > kScratchBytes)
        return fail(MGI_EUNSUPPORTED, "this call needs " + std::to_string(ws.total) +
                                          " bytes of split workspace, more than the " +
                                          std::to_string(kScratchBytes) +
                                          " bytes of mgi_paged_decode_noalloc's scratch; "
                                          "use mgi_paged_decode with a workspace");
      const int rc = scratch_for_stream(static_cast<hipStream_t>(stream), &workspace);
      if (rc != MGI_OK) return rc;
      workspace_bytes = kScratchBytes;
    }
    if (!workspace) return fail(MGI_EWORKSPACE, "workspace required for split-context pass");
    if (workspace_bytes < ws.total)
      return fail(MGI_EWORKSPACE, "workspace smaller than mgi_paged_decode_workspace_bytes()");
    if (!aligned16(workspace)) return fail(MGI_EINVAL, "workspace must be 16-byte aligned");
    a.ws_acc = static_cast<float*>(workspace);
    a.ws_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) + ws.ml_offset);
    if (sp.bal_waves > 0) {
      a.bal_waves = sp.bal_waves;
      a.bal_min_blocks = sp.bal_min_blocks;
      a.bal_tier1_16ths = sp.bal_tier1_16ths;
      a.bal_tier2 = sp.bal_tier2;
      a.bal_claims = sp.bal_waves * (1 + sp.bal_tier2);
      a.ws_cinc = reinterpret_cast<int*>(static_cast<char*>(workspace) + ws.cinc_offset);
      a.ws_ticket = reinterpret_cast<int*>(static_cast<char*>(workspace) + ws.ticket_offset);
    }
  }

  if (ap) {
    const int64_t* ks = ap->kn_strides;
    const int64_t* vs = ap->vn_strides;
    const bool fuse = plan.path == DecodePath::kFast && ap->new_dtype == dtype && ks[2] == 1 &&
                      vs[2] == 1 && aligned16(ap->k_new) && aligned16(ap->v_new) &&
                      mult16(ks[0], eb) && mult16(ks[1], eb) && mult16(vs[0], eb) && mult16(vs[1], eb);
    if (fuse) {
      a.kw = static_cast<char*>(ap->k_pool) + layer_idx * k_pool_strides[0] * eb;
      a.vw = static_cast<char*>(ap->v_pool) + layer_idx * v_pool_strides[0] * eb;
      a.kn = ap->k_new;
      a.vn = ap->v_new;
      a.kn_sb = ks[0];
      a.kn_sh = ks[1];
      a.vn_sb = vs[0];
      a.vn_sh = vs[1];
      a.slots = ap->slots;
      a.sl_s = ap->slot_stride;
      a.sl_i64 = ap->slot_itype == MGI_I64;
    } else {
      const int rc = launch_append(*ap, k_pool_strides, v_pool_strides, dtype, B, H, D, S, N, layer_idx,
                                   static_cast<hipStream_t>(stream));
      if (rc != MGI_OK) return rc;
    }
  }

  // The merge runs one workgroup per (sequence, head group). When those are
  // few, each folds many partials in a chain of dependent loads; give it up
  // to 8 wavefronts, so the merge has about two per CU. Measured on MI355X
  // at B=8 x 32k-128k contexts with 4 heads: one wavefront per workgroup took
  // 43-55 us of a 277 us call.
  a.merge_waves = 1;
  if (plan.path == DecodePath::kFast) {
    const int64_t groups = (H + 64 / plan.lanes_per_head - 1) / (64 / plan.lanes_per_head);
    while (a.merge_waves < 8 && B * groups * a.merge_waves < 2 * (int64_t)device_cus()) a.merge_waves *= 2;
  }
  const hipError_t e = launch_paged_decode(a, dtype, plan, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MGI_ELAUNCH, std::string("launch failed: ") + hipGetErrorString(e));
  return MGI_OK;
}

}  // namespace

extern "C" {

int mgi_paged_decode(void* out, const int64_t* out_strides, const void* q,
                     const int64_t* q_strides, const void* k_pool, const void* v_pool,
                     const int64_t* k_pool_strides, const int64_t* v_pool_strides, int dtype,
                     const void* block_tables, const int64_t* bt_strides, int bt_itype,
                     const void* context_lens, int64_t cl_stride, int cl_itype, int64_t B,
                     int64_t H, int64_t D, int64_t S, int64_t N, int64_t M, int64_t L,
                     int64_t layer_idx, float scale, int64_t split_tokens, void* workspace,
                     size_t workspace_bytes, void* stream) {
  return paged_decode_impl(out, out_strides, q, q_strides, k_pool, v_pool, k_pool_strides,
                           v_pool_strides, dtype, block_tables, bt_strides, bt_itype, context_lens,
                           cl_stride, cl_itype, B, H, D, S, N, M, L, layer_idx, scale, split_tokens,
                           workspace, workspace_bytes, false, nullptr, stream);
}

int mgi_paged_decode_append(void* out, const int64_t* out_strides, const void* q,
                            const int64_t* q_strides, void* k_pool, void* v_pool,
                            const int64_t* k_pool_strides, const int64_t* v_pool_strides, int dtype,
                            const void* k_new, const void* v_new, const int64_t* k_new_strides,
                            const int64_t* v_new_strides, int new_dtype, const void* slot_mapping,
                            int64_t slot_stride, int slot_itype, const void* block_tables,
                            const int64_t* bt_strides, int bt_itype, const void* context_lens,
                            int64_t cl_stride, int cl_itype, int64_t B, int64_t H, int64_t D,
                            int64_t S, int64_t N, int64_t M, int64_t L, int64_t layer_idx,
                            float scale, int64_t split_tokens, void* workspace,
                            size_t workspace_bytes, void* stream) {
  const AppendSpec ap{k_pool, v_pool, k_new, v_new, k_new_strides, v_new_strides, new_dtype,
                      slot_mapping, slot_stride, slot_itype};
  return paged_decode_impl(out, out_strides, q, q_strides, k_pool, v_pool, k_pool_strides,
                           v_pool_strides, dtype, block_tables, bt_strides, bt_itype, context_lens,
                           cl_stride, cl_itype, B, H, D, S, N, M, L, layer_idx, scale, split_tokens,
                           workspace, workspace_bytes, false, &ap, stream);
}

int mgi_paged_decode_noalloc(void* out, const int64_t* out_strides, const void* q,
                             const int64_t* q_strides, const void* k_pool, const void* v_pool,
                             const int64_t* k_pool_strides, const int64_t* v_pool_strides,
                             int dtype, const void* block_tables, const int64_t* bt_strides,
                             int bt_itype, const void* context_lens, int64_t cl_stride,
                             int cl_itype, int64_t B, int64_t H, int64_t D, int64_t S, int64_t N,
                             int64_t M, int64_t L, int64_t layer_idx, float scale,
                             int64_t split_tokens, void* stream) {
  return paged_decode_impl(out, out_strides, q, q_strides, k_pool, v_pool, k_pool_strides,
                           v_pool_strides, dtype, block_tables, bt_strides, bt_itype, context_lens,
                           cl_stride, cl_itype, B, H, D, S, N, M, L, layer_idx, scale, split_tokens,
                           nullptr, 0, true, nullptr, stream);
}

int mgi_kv_append(void* k_pool, void* v_pool, const int64_t* k_pool_strides,
                  const int64_t* v_pool_strides, int pool_dtype, const void* k_new,
                  const void* v_new, const int64_t* k_new_strides, const int64_t* v_new_strides,
                  int new_dtype, const void* slot_mapping, int64_t slot_stride, int slot_itype,
                  int64_t T, int64_t H, int64_t D, int64_t S, int64_t N, int64_t L,
                  int64_t layer_idx, void* stream) {
  using namespace mgi;
  g_err.clear();
  if (T < 0) return fail(MGI_EINVAL, "row count must be non-negative");
  if (T == 0) return MGI_OK;
  if (!k_pool || !v_pool) return fail(MGI_EINVAL, "null tensor pointer");
  if (!k_pool_strides || !v_pool_strides) return fail(MGI_EINVAL, "null stride array");
  if (H <= 0 || D <= 0 || S <= 0 || N <= 0 || L <= 0)
    return fail(MGI_EINVAL, "pool dimensions must be nonzero");
  if (layer_idx < 0 || layer_idx >= L) return fail(MGI_EINVAL, "layer_idx outside KV pool");
  if (!valid_dtype(pool_dtype)) return fail(MGI_EINVAL, "unknown dtype code");
  if (!nonneg(k_pool_strides, 5) || !nonneg(v_pool_strides, 5)) return fail(MGI_EINVAL, "strides must be non-negative");
  const AppendSpec ap{k_pool, v_pool, k_new, v_new, k_new_strides, v_new_strides, new_dtype,
                      slot_mapping, slot_stride, slot_itype};
  const int rc = check_append(ap, pool_dtype, T);
  if (rc != MGI_OK) return rc;
  return launch_append(ap, k_pool_strides, v_pool_strides, pool_dtype, T, H, D, S, N, layer_idx,
                       static_cast<hipStream_t>(stream));
}

int mgi_paged_prefill(void* out, const int64_t* out_strides, const void* q,
                      const int64_t* q_strides, const void* k_pool, const void* v_pool,
                      const int64_t* k_pool_strides, const int64_t* v_pool_strides, int dtype,
                      const void* block_table, int64_t bt_stride, int bt_itype, int64_t n_blocks,
                      int64_t start_pos, int64_t T, int64_t H, int64_t D, int64_t S, int64_t N,
                      int64_t L, int64_t layer_idx, float scale, void* workspace,
                      size_t workspace_bytes, void* stream) {
  using namespace mgi;
  g_err.clear();
  if (T < 0) return fail(MGI_EINVAL, "row count must be non-negative");
  if (T == 0) return MGI_OK;
  if (!out || !q || !k_pool || !v_pool || !block_table) return fail(MGI_EINVAL, "null tensor pointer");
  if (!out_strides || !q_strides || !k_pool_strides || !v_pool_strides)
    return fail(MGI_EINVAL, "null stride array");
  if (H <= 0 || D <= 0) return fail(MGI_EINVAL, "q dimensions must be nonzero");
  if (S <= 0 || N <= 0 || L <= 0) return fail(MGI_EINVAL, "pool dimensions must be nonzero");
  if (layer_idx < 0 || layer_idx >= L) return fail(MGI_EINVAL, "layer_idx outside KV pool");
  if (start_pos < 0) return fail(MGI_EINVAL, "start_pos must be non-negative");
  if (n_blocks < (start_pos + T + S - 1) / S)
    return fail(MGI_EINVAL, "block table shorter than ceil((start_pos + T) / S)");
  if (!valid_dtype(dtype)) return fail(MGI_EINVAL, "unknown dtype code");
  if (!valid_itype(bt_itype)) return fail(MGI_EINVAL, "block_table must be int32 or int64");
  if (!std::isfinite(scale)) return fail(MGI_EINVAL, "scale must be finite");
  if (!nonneg(out_strides, 3) || !nonneg(q_strides, 3) || !nonneg(k_pool_strides, 5) ||
      !nonneg(v_pool_strides, 5) || bt_stride < 0)
    return fail(MGI_EINVAL, "strides must be non-negative");
  if (start_pos + T >= (int64_t(1) << 31)) return fail(MGI_EUNSUPPORTED, "start_pos + T must be < 2^31");
  if (H > kMaxGridYZ) return fail(MGI_EUNSUPPORTED, "more than 65535 heads");
  if (((T + 31) / 32) * H > (int64_t(1) << 24))
    return fail(MGI_EUNSUPPORTED, "chunk rows x heads too large for one launch");
  if (D > 512) return fail(MGI_EUNSUPPORTED, "head_dim larger than 512");

  const int64_t eb = dtype_bytes(dtype);
  const char* kbase = static_cast<const char*>(k_pool) + layer_idx * k_pool_strides[0] * eb;
  const char* vbase = static_cast<const char*>(v_pool) + layer_idx * v_pool_strides[0] * eb;
  const int dp = prefill_head_dim_bucket(dtype != MGI_F32, (int)D);

  // Matrix-core path: head dim a multiple of one 16-byte chunk
  // within the padded bucket, unit head-dim strides, 16-byte aligned rows.
  const bool mfma = dp != 0 && D % (16 / eb) == 0 && q_strides[2] == 1 && out_strides[2] == 1 &&
                    k_pool_strides[4] == 1 && v_pool_strides[4] == 1 && aligned16(q) &&
                    aligned16(out) && aligned16(kbase) && aligned16(vbase) &&
                    mult16(q_strides[0], eb) && mult16(q_strides[1], eb) &&
                    mult16(out_strides[0], eb) && mult16(out_strides[1], eb) &&
                    mult16(k_pool_strides[1], eb) && mult16(k_pool_strides[2], eb) &&
                    mult16(k_pool_strides[3], eb) && mult16(v_pool_strides[1], eb) &&
                    mult16(v_pool_strides[2], eb) && mult16(v_pool_strides[3], eb) &&
                    N < (int64_t(1) << 31);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (mfma) {
    PrefillArgs a{};
    a.out = out;
    a.o_st = out_strides[0];
    a.o_sh = out_strides[1];
    a.q = q;
    a.q_st = q_strides[0];
    a.q_sh = q_strides[1];
    a.k = kbase;
    a.v = vbase;
    a.k_sn = k_pool_strides[1];
    a.k_ss = k_pool_strides[2];
    a.k_sh = k_pool_strides[3];
    a.v_sn = v_pool_strides[1];
    a.v_ss = v_pool_strides[2];
    a.v_sh = v_pool_strides[3];
    a.bt = block_table;
    a.bt_s = bt_stride;
    a.bt_i64 = bt_itype == MGI_I64;
    a.start = (int)start_pos;
    a.T = (int)T;
    a.H = (int)H;
    a.D = (int)D;
    a.S = (int)S;
    a.s_shift = (S & (S - 1)) == 0 ? __builtin_ctzll((unsigned long long)S) : -1;
    a.N = N;
    a.scale_log2 = scale * 1.4426950408889634f;
    // Four wavefronts of 16 query rows share each staged K/V tile; chunks of
    // at most 32 rows use two. (Two-wave workgroups for grids that leave CUs
    // empty measured slower on MI355X: 19.3 against 16.7 us for a 512-row
    // bf16 chunk of 16 heads, as each thread then stages twice the tile.)
    a.cus = device_cus();
    const int waves = T <= 32 ? 2 : 4;
    const PrefillWorkspace pw = prefill_workspace(start_pos, T, H, D, dtype);
    if (pw.part_keys > 0) {
      if (!workspace) return fail(MGI_EWORKSPACE, "workspace required for the split-key pass");
      if (workspace_bytes < pw.total)
        return fail(MGI_EWORKSPACE, "workspace smaller than mgi_paged_prefill_workspace_bytes()");
      if (!aligned16(workspace)) return fail(MGI_EINVAL, "workspace must be 16-byte aligned");
      a.part_keys = (int)pw.part_keys;
      a.max_parts = (int)pw.max_parts;
      a.ws_acc = static_cast<float*>(workspace);
      a.ws_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) + pw.ml_offset);
    }
    e = launch_paged_prefill(a, dtype, dp, waves, 1, st);
    if (e == hipSuccess && pw.part_keys > 0) {
      // Rows whose keys span several partitions: the decode merge in
      // partition mode, row i at context start_pos + i + 1.
      DecodeArgs m{};
      m.out = out;
      m.o_sb = out_strides[0];
      m.o_sh = out_strides[1];
      m.o_sd = out_strides[2];
      m.cl = nullptr;
      m.ctx_base = start_pos;
      m.B = (int)T;
      m.H = (int)H;
      m.D = (int)D;
      m.S = (int)S;
      m.M = (int)((start_pos + T + S - 1) / S);
      m.N = N;
      m.part_tokens = (int)pw.part_keys;
      m.max_parts = (int)pw.max_parts;
      m.ws_acc = a.ws_acc;
      m.ws_ml = a.ws_ml;
      const int lph = next_pow2_at_least4(D / 8);
      const int64_t groups = (H + 64 / lph - 1) / (64 / lph);
      m.merge_waves = 1;
      while (m.merge_waves < 8 && T * groups * m.merge_waves < 2 * (int64_t)device_cus()) m.merge_waves *= 2;
      e = launch_paged_merge(m, dtype, lph, st);
    }
  } else {
    // Any other shape: the chunk as T single-query rows of the generic decode
    // kernel, sharing one table row, with context lengths start_pos + t + 1.
    if (T > kMaxGridYZ) return fail(MGI_EUNSUPPORTED, "chunk longer than 65535 rows for this shape");
    if (n_blocks * S >= (int64_t(1) << 31)) return fail(MGI_EUNSUPPORTED, "n_blocks*S must be < 2^31");
    DecodeArgs a{};
    a.out = out;
    a.o_sb = out_strides[0];
    a.o_sh = out_strides[1];
    a.o_sd = out_strides[2];
    a.q = q;
    a.q_sb = q_strides[0];
    a.q_sh = q_strides[1];
    a.q_sd = q_strides[2];
    a.k = kbase;
    a.v = vbase;
    a.k_sn = k_pool_strides[1];
    a.k_ss = k_pool_strides[2];
    a.k_sh = k_pool_strides[3];
    a.k_sd = k_pool_strides[4];
    a.v_sn = v_pool_strides[1];
    a.v_ss = v_pool_strides[2];
    a.v_sh = v_pool_strides[3];
    a.v_sd = v_pool_strides[4];
    a.bt = block_table;
    a.bt_sb = 0;
    a.bt_sm = bt_stride;
    a.cl = nullptr;
    a.ctx_base = start_pos;
    a.bt_i64 = bt_itype == MGI_I64;
    a.B = (int)T;
    a.H = (int)H;
    a.D = (int)D;
    a.S = (int)S;
    a.M = (int)n_blocks;
    a.N = N;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.part_tokens = (int)(n_blocks * S);
    a.max_parts = 1;
    DecodePlan plan{};
    plan.path = DecodePath::kGeneric;
    e = launch_paged_decode(a, dtype, plan, st);
  }
  if (e != hipSuccess) return fail(MGI_ELAUNCH, std::string("launch failed: ") + hipGetErrorString(e));
  return MGI_OK;
}

}  // extern "C"
