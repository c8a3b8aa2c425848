// C ABI of libmi_fa2.so: argument validation, split-KV sizing and kernel dispatch.
// Declarations and the contract of every entry point are in include/mi_fa2.h.
#include "mi_fa2.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>

#include "fa2_common.h"

namespace mi_fa2 {
hipError_t launch_prefill(const FwdParams& p, int dtype, int mode, int max_seqlen_q,
                          hipStream_t stream);
hipError_t launch_decode(const FwdParams& p, int dtype, int mode, hipStream_t stream);
hipError_t launch_general(const FwdParams& p, int dtype, int d, int dv, hipStream_t stream);
hipError_t launch_merge(const MergeParams& p, int out_dtype, hipStream_t stream);
hipError_t launch_rope_kv(const RopeParams& p, int dtype, hipStream_t stream);
hipError_t launch_sample(const SampleParams& p, int dtype, hipStream_t stream);
int sample_chunks(int vocab);
hipError_t launch_step_meta(const StepMetaParams& p, hipStream_t stream);
hipError_t launch_add_rmsnorm(const ModelOpParams& p, int dtype, hipStream_t stream);
hipError_t launch_silu_mul(const ModelOpParams& p, int dtype, hipStream_t stream);
}  // namespace mi_fa2

using mi_fa2::FwdParams;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return MI_FA2_OK;
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// Decode work split: the kernel cuts every (row, kv head) item into 128-key chunks and gives each
// of its work-groups an equal contiguous share of all the chunks (stream-K); an item cut by a share
// boundary leaves one partial per work-group touching it.  Work-groups launched: as many as fit on
// the device's CUs at once (4 waves each: 2 per CU for the dense walk at 2 waves per SIMD, 3 per CU
// for the paged walk at 3 waves per SIMD; 512 and 768 on the 256 CUs of MI355X), never more than
// there are chunks.  MI_FA2_DECODE_WGS overrides it, for tuning sweeps.
constexpr int kDecodeChunk = 128;

// What the launches are sized from: the device's compute units and XCDs (each XCD has its own L2,
// and work-group w of a launch runs on XCD w % XCDs).  MI355X: 256 CUs in 8 XCDs; a partitioned
// device reports its own share.  The XCD mapping of the prefill grid needs a power of two; any
// other count maps as if there were one XCD (correct, only the L2 affinity is lost).
struct Plan {
  int cus, xcds, xcd_log2, decode_wgs_paged, decode_wgs_dense;
};

int forced_decode_wgs() {
  static const int forced = [] {
    const char* env = std::getenv("MI_FA2_DECODE_WGS");
    const int v = env ? std::atoi(env) : 0;
    return v > 0 ? v : 0;
  }();
  return forced;
}

Plan make_plan(int cus, int xcds) {
  Plan pl{};
  pl.cus = std::max(1, cus);
  pl.xcds = std::max(1, xcds);
  pl.xcd_log2 = 0;
  while ((2 << pl.xcd_log2) <= pl.xcds && pl.xcd_log2 < 6) ++pl.xcd_log2;
  if ((1 << pl.xcd_log2) != pl.xcds) pl.xcd_log2 = 0;
  const int forced = forced_decode_wgs();
  pl.decode_wgs_paged = forced ? forced : 3 * pl.cus;
  pl.decode_wgs_dense = forced ? forced : 2 * pl.cus;
  return pl;
}

constexpr int kMaxDevices = 64;
std::once_flag g_plan_once[kMaxDevices];
Plan g_plan[kMaxDevices];
hipError_t g_plan_err[kMaxDevices];

// The current device's plan, read once per device.
int plan_of_current_device(Plan* out) {
  int dev = -1;
  const hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess)
    return fail(MI_FA2_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MI_FA2_ERR_UNSUPPORTED, "device %d: the device table holds %d devices", dev,
                kMaxDevices);
  std::call_once(g_plan_once[dev], [dev] {
    int cus = 0, xcds = 0;
    g_plan_err[dev] = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (g_plan_err[dev] == hipSuccess)
      g_plan_err[dev] = hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, dev);
    g_plan[dev] = make_plan(cus, xcds);
  });
  if (g_plan_err[dev] != hipSuccess)
    return fail(MI_FA2_ERR_LAUNCH, "reading device %d's CU / XCD counts failed: %s", dev,
                hipGetErrorString(g_plan_err[dev]));
  *out = g_plan[dev];
  return MI_FA2_OK;
}

// The clock probe set by mi_fa2_set_clock_probe (measurement only; null: off).
std::atomic<uint64_t*> g_clock_probe{nullptr};

// Fills the launch's device fields (CU count, XCD mapping, clock probe) from the current device.
int set_device(FwdParams& p, Plan* plan = nullptr) {
  Plan pl;
  if (int rc = plan_of_current_device(&pl)) return rc;
  p.n_cus = pl.cus;
  p.xcd_log2 = pl.xcd_log2;
  p.clock_probe = g_clock_probe.load(std::memory_order_relaxed);
  if (plan) *plan = pl;
  return MI_FA2_OK;
}

// The split decode kernel serves one query per row, up to 16 query heads per kv head (the N of its
// 16x16 MFMA) and up to 8192 rows (its row prefix sum lives in LDS); anything else runs through
// the prefill kernel, which handles a single query row too.
constexpr int kMaxDecodeBatch = 8192;
bool uses_decode(int64_t seqlen_q, int64_t group, int64_t batch) {
  return seqlen_q == 1 && group <= 16 && batch <= kMaxDecodeBatch;
}

// The decode kernel reads a 16-token run through a buffer resource of 32-bit byte offsets.
int check_decode_strides(const FwdParams& p) {
  const int64_t lim = int64_t(1) << 26;  // 16 rows x 2 bytes x stride < 2^31
  if (p.k_st < 0 || p.v_st < 0 || p.k_st >= lim || p.v_st >= lim)
    return fail(MI_FA2_ERR_UNSUPPORTED, "k/v token strides %lld / %lld: at most 2^26 - 1 elements",
                (long long)p.k_st, (long long)p.v_st);
  return MI_FA2_OK;
}

// The prefill kernel loads up to 64 K/V rows through one buffer resource (32-bit byte extent
// rows x 2 bytes x stride) and adds 32-row offsets of 32-bit bytes: token strides stay below 2^24.
int check_prefill_strides(int64_t k_st, int64_t v_st) {
  const int64_t lim = int64_t(1) << 24;  // 64 rows x 2 bytes x stride < 2^31
  if (k_st < 0 || v_st < 0 || k_st >= lim || v_st >= lim)
    return fail(MI_FA2_ERR_UNSUPPORTED, "k/v token strides %lld / %lld: at most 2^24 - 1 elements",
                (long long)k_st, (long long)v_st);
  return MI_FA2_OK;
}

int decode_work_groups(const Plan& pl, int64_t batch, int64_t heads_kv, int64_t max_kv,
                       bool paged) {
  const int64_t chunks = batch * heads_kv * std::max<int64_t>(1, (max_kv + kDecodeChunk - 1) / kDecodeChunk);
  const int64_t want = paged ? pl.decode_wgs_paged : pl.decode_wgs_dense;
  return (int)std::max<int64_t>(1, std::min(want, chunks));
}

// Partial slots per (row, query head): at most one per chunk of the longest row.
int decode_splits(int64_t max_kv) {
  return max_kv > 0 ? (int)((max_kv + kDecodeChunk - 1) / kDecodeChunk) : 1;
}

// Workspace of a split decode: fp32 partial O [B][Hq][splits][128], m [B][Hq][splits],
// l [B][Hq][splits], then the int32 partial count of every (row, kv head) item [B][Hkv].
size_t decode_workspace(int64_t batch, int64_t heads_q, int64_t heads_kv, int64_t max_kv) {
  const int splits = decode_splits(max_kv);
  if (splits <= 1) return 0;
  return (size_t)batch * heads_q * splits * (mi_fa2::kHeadDim + 2) * sizeof(float) +
         (size_t)batch * heads_kv * sizeof(int32_t);
}

void set_workspace(FwdParams& p, void* workspace) {
  float* ws = static_cast<float*>(workspace);
  const size_t slots = (size_t)p.B * p.Hq * p.max_splits;
  p.ws_o = ws;
  p.ws_m = ws + slots * mi_fa2::kHeadDim;
  p.ws_l = p.ws_m + slots;
  p.ws_np = reinterpret_cast<int32_t*>(p.ws_l + slots);
}

int check_common(int32_t dtype, int32_t batch, int32_t heads_q, int32_t heads_kv,
                 int32_t head_dim) {
  if (dtype != MI_FA2_BF16 && dtype != MI_FA2_FP16)
    return fail(MI_FA2_ERR_UNSUPPORTED, "dtype %d is not bf16 (0) or fp16 (1)", dtype);
  if (batch < 0 || heads_q <= 0 || heads_kv <= 0)
    return fail(MI_FA2_ERR_INVALID, "bad sizes: batch=%d heads_q=%d heads_kv=%d", batch, heads_q,
                heads_kv);
  if (heads_q % heads_kv != 0)
    return fail(MI_FA2_ERR_INVALID, "heads_q (%d) must be a multiple of heads_kv (%d)", heads_q,
                heads_kv);
  if (head_dim != mi_fa2::kHeadDim)
    return fail(MI_FA2_ERR_UNSUPPORTED, "head_dim %d: the kernels are built for head_dim 128",
                head_dim);
  return MI_FA2_OK;
}

int check_tensor(const char* name, const void* ptr, const int64_t* strides, int n_outer) {
  if (!ptr) return fail(MI_FA2_ERR_INVALID, "%s is NULL", name);
  if (!aligned16(ptr)) return fail(MI_FA2_ERR_INVALID, "%s is not 16-byte aligned", name);
  if (!strides) return fail(MI_FA2_ERR_INVALID, "%s strides are NULL", name);
  for (int i = 0; i < n_outer; ++i)
    if (strides[i] % 8 != 0)
      return fail(MI_FA2_ERR_INVALID, "%s stride[%d] = %lld is not a multiple of 8 elements", name,
                  i, (long long)strides[i]);
  return MI_FA2_OK;
}

// K and V rows are loaded through buffer resources whose extent is (rows) x (token stride): a
// token stride below the head dim would cut the last row short (and rows would overlap).
int check_pitch(const char* name, int64_t token_stride) {
  if (token_stride < mi_fa2::kHeadDim)
    return fail(MI_FA2_ERR_INVALID, "%s token stride %lld is below head_dim %d (rows overlap)", name,
                (long long)token_stride, mi_fa2::kHeadDim);
  return MI_FA2_OK;
}

int launched(hipError_t err) {
  if (err != hipSuccess)
    return fail(MI_FA2_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return ok();
}

void set_lse(FwdParams& p, float* lse, const int64_t* s, int n) {
  p.lse = lse;
  if (!lse) return;
  if (n == 3) {
    p.l_sb = s[0];
    p.l_sh = s[1];
    p.l_st = s[2];
  } else {  // varlen: (head, token)
    p.l_sh = s[0];
    p.l_st = s[1];
  }
}

// Scratch of the no-allocation entry point (mi_fa2_fwd_paged_noalloc): the split-decode
// workspace as a device array of fixed size, which every GPU the library runs on holds until the
// process ends.  Host code never passes `scratch` itself to a kernel (on the host that name is a
// stand-in, not the device address): the address is looked up once per device with
// hipGetSymbolAddress, with that device current, and kept.  Calls on one GPU share its array, so
// calls that overlap in time on one GPU (different streams) race.  Nothing in it needs clearing:
// every partial and count the combine reads is written by the same launch.
constexpr size_t kScratchBytes = 32u << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

int scratch_of_current_device(void** out) {
  int dev = -1;
  const hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess)
    return fail(MI_FA2_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MI_FA2_ERR_UNSUPPORTED, "device %d: the scratch table holds %d devices", dev,
                kMaxDevices);
  std::call_once(g_scratch_once[dev], [dev] {
    g_scratch_err[dev] = hipGetSymbolAddress(&g_scratch_ptr[dev], HIP_SYMBOL(scratch));
  });
  if (g_scratch_err[dev] != hipSuccess || !g_scratch_ptr[dev])
    return fail(MI_FA2_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(g_scratch_err[dev]));
  *out = g_scratch_ptr[dev];
  return MI_FA2_OK;
}

// The paged forward behind mi_fa2_fwd_paged (caller's workspace) and mi_fa2_fwd_paged_noalloc
// (the library's static scratch: use_scratch).
int fwd_paged(int32_t dtype, const void* q, const void* k_pool, const void* v_pool, void* o,
              float* lse, const int32_t* block_table, int64_t block_table_stride,
              const int32_t* kv_lens, int32_t batch, int32_t heads_q, int32_t heads_kv,
              int32_t seqlen_q, int32_t max_kv_len, int32_t head_dim, int32_t block_size,
              int32_t num_blocks, const int64_t* q_strides, const int64_t* pool_strides,
              const int64_t* o_strides, const int64_t* lse_strides, int32_t is_causal,
              float sm_scale, void* workspace, size_t workspace_bytes, bool use_scratch,
              mi_fa2_stream_t stream) {
  if (int rc = check_common(dtype, batch, heads_q, heads_kv, head_dim)) return rc;
  if (seqlen_q < 0 || max_kv_len < 0)
    return fail(MI_FA2_ERR_INVALID, "bad lengths: seqlen_q=%d max_kv_len=%d", seqlen_q,
                max_kv_len);
  if (block_size < 16 || (block_size & (block_size - 1)))
    return fail(MI_FA2_ERR_UNSUPPORTED, "block_size %d is not a power of two >= 16", block_size);
  if (num_blocks < 0) return fail(MI_FA2_ERR_INVALID, "num_blocks %d < 0", num_blocks);
  if (batch == 0 || seqlen_q == 0) return ok();
  if (!kv_lens) return fail(MI_FA2_ERR_INVALID, "kv_lens is NULL");
  if (max_kv_len > 0 && !block_table) return fail(MI_FA2_ERR_INVALID, "block_table is NULL");
  if (int rc = check_tensor("q", q, q_strides, 3)) return rc;
  if (int rc = check_tensor("o", o, o_strides, 3)) return rc;
  if (int rc = check_tensor("k_pool", k_pool, pool_strides, 2)) return rc;
  if (int rc = check_tensor("v_pool", v_pool, pool_strides, 2)) return rc;
  if (int rc = check_pitch("pool", pool_strides[0])) return rc;
  if (lse && !lse_strides) return fail(MI_FA2_ERR_INVALID, "lse strides are NULL");

  FwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k_pool);
  p.v = static_cast<const uint16_t*>(v_pool);
  p.o = static_cast<uint16_t*>(o);
  p.kv_lens = kv_lens;
  p.block_table = block_table;
  p.bt_stride = block_table_stride;
  p.block_size = block_size;
  p.num_blocks = num_blocks;
  p.q_sb = q_strides[0], p.q_sh = q_strides[1], p.q_st = q_strides[2];
  p.o_sb = o_strides[0], p.o_sh = o_strides[1], p.o_st = o_strides[2];
  p.k_st = pool_strides[0], p.k_sh = pool_strides[1];
  p.v_st = pool_strides[0], p.v_sh = pool_strides[1];
  set_lse(p, lse, lse_strides, 3);
  p.B = batch;
  p.Hq = heads_q;
  p.Hkv = heads_kv;
  p.group = heads_q / heads_kv;
  p.T = seqlen_q;
  p.S = max_kv_len;
  p.causal = is_causal ? 1 : 0;
  p.scale_log2 = sm_scale * mi_fa2::kLog2e;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // Every argument is checked before the device is looked at (its CU / XCD counts size the grid).
  Plan plan;

  if (uses_decode(seqlen_q, p.group, batch)) {
    p.max_splits = decode_splits(max_kv_len);
    const size_t need = decode_workspace(batch, heads_q, heads_kv, max_kv_len);
    if (need && use_scratch) {
      if (need > kScratchBytes)
        return fail(MI_FA2_ERR_WORKSPACE,
                    "decode needs %zu scratch bytes; the no-allocation entry point holds at most "
                    "%zu (use mi_fa2_fwd_paged with a workspace)", need, kScratchBytes);
      if (int rc = scratch_of_current_device(&workspace)) return rc;
      workspace_bytes = kScratchBytes;
    }
    if (need) {
      if (!workspace || workspace_bytes < need)
        return fail(MI_FA2_ERR_WORKSPACE, "decode needs %zu workspace bytes, got %zu", need,
                    workspace ? workspace_bytes : (size_t)0);
      set_workspace(p, workspace);
    }
    if (int rc = check_decode_strides(p)) return rc;
    if (int rc = set_device(p, &plan)) return rc;
    p.n_wg = decode_work_groups(plan, batch, heads_kv, max_kv_len, true);
    return launched(mi_fa2::launch_decode(p, dtype, mi_fa2::kPaged, s));
  }
  if (int rc = check_prefill_strides(p.k_st, p.v_st)) return rc;
  if (int rc = set_device(p, &plan)) return rc;
  return launched(mi_fa2::launch_prefill(p, dtype, mi_fa2::kPaged, seqlen_q, s));
}

}  // namespace

extern "C" {

const char* mi_fa2_version(void) { return "mi_fa2 0.1.0 gfx950"; }

const char* mi_fa2_last_error(void) { return g_err; }

int mi_fa2_launch_plan(int32_t num_cus, int32_t num_xcds, mi_fa2_plan* out) {
  if (!out) return fail(MI_FA2_ERR_INVALID, "out is NULL");
  Plan pl;
  if (num_cus > 0) {
    pl = make_plan(num_cus, num_xcds);
  } else if (int rc = plan_of_current_device(&pl)) {
    return rc;
  }
  out->num_cus = pl.cus;
  out->num_xcds = pl.xcds;
  out->xcds_mapped = 1 << pl.xcd_log2;
  out->decode_work_groups_paged = pl.decode_wgs_paged;
  out->decode_work_groups_dense = pl.decode_wgs_dense;
  out->prefill_one_stream_min_work_groups = mi_fa2::prefill_one_stream_min_grid(pl.cus);
  out->prefill_one_stream_max_keys = mi_fa2::kPrefillOneStreamMaxKeys;
  return ok();
}

int mi_fa2_set_clock_probe(uint64_t* probe) {
  if (reinterpret_cast<uintptr_t>(probe) % 8)
    return fail(MI_FA2_ERR_INVALID, "probe is not 8-byte aligned");
  g_clock_probe.store(probe, std::memory_order_relaxed);
  return ok();
}

size_t mi_fa2_fwd_workspace_size(int32_t batch, int32_t heads_q, int32_t heads_kv,
                                 int32_t seqlen_q, int32_t seqlen_k, int32_t head_dim) {
  (void)head_dim;
  if (heads_kv <= 0 || heads_q % heads_kv || !uses_decode(seqlen_q, heads_q / heads_kv, batch))
    return 0;
  return decode_workspace(batch, heads_q, heads_kv, seqlen_k);
}

int mi_fa2_fwd(int32_t dtype, const void* q, const void* k, const void* v, void* o, float* lse,
               const int32_t* kv_lens, int32_t batch, int32_t heads_q, int32_t heads_kv,
               int32_t seqlen_q, int32_t seqlen_k, int32_t head_dim, const int64_t* q_strides,
               const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
               const int64_t* lse_strides, int32_t is_causal, float sm_scale, void* workspace,
               size_t workspace_bytes, mi_fa2_stream_t stream) {
  if (int rc = check_common(dtype, batch, heads_q, heads_kv, head_dim)) return rc;
  if (seqlen_q < 0 || seqlen_k < 0)
    return fail(MI_FA2_ERR_INVALID, "bad lengths: seqlen_q=%d seqlen_k=%d", seqlen_q, seqlen_k);
  if (batch == 0 || seqlen_q == 0) return ok();
  if (int rc = check_tensor("q", q, q_strides, 3)) return rc;
  if (int rc = check_tensor("o", o, o_strides, 3)) return rc;
  if (seqlen_k > 0) {
    if (int rc = check_tensor("k", k, k_strides, 3)) return rc;
    if (int rc = check_tensor("v", v, v_strides, 3)) return rc;
    if (int rc = check_pitch("k", k_strides[2])) return rc;
    if (int rc = check_pitch("v", v_strides[2])) return rc;
  }
  if (lse && !lse_strides) return fail(MI_FA2_ERR_INVALID, "lse strides are NULL");

  FwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<uint16_t*>(o);
  p.kv_lens = kv_lens;
  p.q_sb = q_strides[0], p.q_sh = q_strides[1], p.q_st = q_strides[2];
  p.o_sb = o_strides[0], p.o_sh = o_strides[1], p.o_st = o_strides[2];
  if (seqlen_k > 0) {
    p.k_sb = k_strides[0], p.k_sh = k_strides[1], p.k_st = k_strides[2];
    p.v_sb = v_strides[0], p.v_sh = v_strides[1], p.v_st = v_strides[2];
  }
  set_lse(p, lse, lse_strides, 3);
  p.B = batch;
  p.Hq = heads_q;
  p.Hkv = heads_kv;
  p.group = heads_q / heads_kv;
  p.T = seqlen_q;
  p.S = seqlen_k;
  p.causal = is_causal ? 1 : 0;
  p.scale_log2 = sm_scale * mi_fa2::kLog2e;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // Every argument is checked before the device is looked at (its CU / XCD counts size the grid).
  Plan plan;

  if (uses_decode(seqlen_q, p.group, batch)) {
    p.max_splits = decode_splits(seqlen_k);
    const size_t need = decode_workspace(batch, heads_q, heads_kv, seqlen_k);
    if (need) {
      if (!workspace || workspace_bytes < need)
        return fail(MI_FA2_ERR_WORKSPACE, "decode needs %zu workspace bytes, got %zu", need,
                    workspace ? workspace_bytes : (size_t)0);
      set_workspace(p, workspace);
    }
    if (int rc = check_decode_strides(p)) return rc;
    if (int rc = set_device(p, &plan)) return rc;
    p.n_wg = decode_work_groups(plan, batch, heads_kv, seqlen_k, false);
    return launched(mi_fa2::launch_decode(p, dtype, mi_fa2::kDense, s));
  }
  if (int rc = check_prefill_strides(p.k_st, p.v_st)) return rc;
  if (int rc = set_device(p, &plan)) return rc;
  return launched(mi_fa2::launch_prefill(p, dtype, mi_fa2::kDense, seqlen_q, s));
}

int mi_fa2_fwd_general(int32_t dtype, const void* q, const void* k, const void* v, void* o,
                       float* lse, const int32_t* kv_lens, int32_t batch, int32_t heads_q,
                       int32_t heads_kv, int32_t seqlen_q, int32_t seqlen_k, int32_t head_dim,
                       int32_t head_dim_v, const int64_t* q_strides, const int64_t* k_strides,
                       const int64_t* v_strides, const int64_t* o_strides,
                       const int64_t* lse_strides, int32_t is_causal, float sm_scale,
                       mi_fa2_stream_t stream) {
  if (dtype != MI_FA2_BF16 && dtype != MI_FA2_FP16 && dtype != MI_FA2_FP32)
    return fail(MI_FA2_ERR_UNSUPPORTED, "dtype %d is not bf16 (0), fp16 (1) or fp32 (2)", dtype);
  auto dim_ok = [](int32_t d) { return d == 16 || d == 32 || d == 64 || d == 128 || d == 256; };
  if (!dim_ok(head_dim) || !dim_ok(head_dim_v))
    return fail(MI_FA2_ERR_UNSUPPORTED,
                "head_dim %d / head_dim_v %d: each must be a power of two from 16 to 256", head_dim,
                head_dim_v);
  if (batch < 0 || heads_q <= 0 || heads_kv <= 0 || heads_q % heads_kv != 0)
    return fail(MI_FA2_ERR_INVALID, "bad sizes: batch=%d heads_q=%d heads_kv=%d", batch, heads_q,
                heads_kv);
  if (batch > 65535 || heads_q > 65535)
    return fail(MI_FA2_ERR_UNSUPPORTED, "batch (%d) and heads_q (%d) are at most 65535", batch,
                heads_q);
  if (seqlen_q < 0 || seqlen_k < 0)
    return fail(MI_FA2_ERR_INVALID, "bad lengths: seqlen_q=%d seqlen_k=%d", seqlen_q, seqlen_k);
  if (batch == 0 || seqlen_q == 0) return ok();
  if (int rc = check_tensor("q", q, q_strides, 3)) return rc;
  if (int rc = check_tensor("o", o, o_strides, 3)) return rc;
  if (seqlen_k > 0) {
    if (int rc = check_tensor("k", k, k_strides, 3)) return rc;
    if (int rc = check_tensor("v", v, v_strides, 3)) return rc;
  }
  if (lse && !lse_strides) return fail(MI_FA2_ERR_INVALID, "lse strides are NULL");

  FwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<uint16_t*>(o);
  p.kv_lens = kv_lens;
  p.q_sb = q_strides[0], p.q_sh = q_strides[1], p.q_st = q_strides[2];
  p.o_sb = o_strides[0], p.o_sh = o_strides[1], p.o_st = o_strides[2];
  if (seqlen_k > 0) {
    p.k_sb = k_strides[0], p.k_sh = k_strides[1], p.k_st = k_strides[2];
    p.v_sb = v_strides[0], p.v_sh = v_strides[1], p.v_st = v_strides[2];
  }
  set_lse(p, lse, lse_strides, 3);
  p.B = batch;
  p.Hq = heads_q;
  p.Hkv = heads_kv;
  p.group = heads_q / heads_kv;
  p.T = seqlen_q;
  p.S = seqlen_k;
  p.causal = is_causal ? 1 : 0;
  p.scale_log2 = sm_scale * mi_fa2::kLog2e;
  if (int rc = set_device(p)) return rc;
  return launched(mi_fa2::launch_general(p, dtype, head_dim, head_dim_v,
                                         reinterpret_cast<hipStream_t>(stream)));
}

int mi_fa2_fwd_varlen(int32_t dtype, const void* q, const void* k, const void* v, void* o,
                      float* lse, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                      int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t max_seqlen_q,
                      int32_t head_dim, const int64_t* q_strides, const int64_t* k_strides,
                      const int64_t* v_strides, const int64_t* o_strides,
                      const int64_t* lse_strides, int32_t is_causal, float sm_scale,
                      mi_fa2_stream_t stream) {
  if (int rc = check_common(dtype, batch, heads_q, heads_kv, head_dim)) return rc;
  if (max_seqlen_q < 0) return fail(MI_FA2_ERR_INVALID, "max_seqlen_q %d < 0", max_seqlen_q);
  if (batch == 0 || max_seqlen_q == 0) return ok();
  if (!cu_seqlens_q || !cu_seqlens_k) return fail(MI_FA2_ERR_INVALID, "cu_seqlens are NULL");
  if (int rc = check_tensor("q", q, q_strides, 2)) return rc;
  if (int rc = check_tensor("k", k, k_strides, 2)) return rc;
  if (int rc = check_tensor("v", v, v_strides, 2)) return rc;
  if (int rc = check_pitch("k", k_strides[0])) return rc;
  if (int rc = check_pitch("v", v_strides[0])) return rc;
  if (int rc = check_tensor("o", o, o_strides, 2)) return rc;
  if (lse && !lse_strides) return fail(MI_FA2_ERR_INVALID, "lse strides are NULL");

  FwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<uint16_t*>(o);
  p.cu_q = cu_seqlens_q;
  p.cu_k = cu_seqlens_k;
  p.q_st = q_strides[0], p.q_sh = q_strides[1];
  p.k_st = k_strides[0], p.k_sh = k_strides[1];
  p.v_st = v_strides[0], p.v_sh = v_strides[1];
  p.o_st = o_strides[0], p.o_sh = o_strides[1];
  set_lse(p, lse, lse_strides, 2);
  p.B = batch;
  p.Hq = heads_q;
  p.Hkv = heads_kv;
  p.group = heads_q / heads_kv;
  p.causal = is_causal ? 1 : 0;
  p.scale_log2 = sm_scale * mi_fa2::kLog2e;
  if (int rc = check_prefill_strides(p.k_st, p.v_st)) return rc;
  if (int rc = set_device(p)) return rc;
  return launched(mi_fa2::launch_prefill(p, dtype, mi_fa2::kVarlen, max_seqlen_q,
                                         reinterpret_cast<hipStream_t>(stream)));
}

size_t mi_fa2_fwd_paged_workspace_size(int32_t batch, int32_t heads_q, int32_t heads_kv,
                                       int32_t seqlen_q, int32_t max_kv_len, int32_t head_dim) {
  return mi_fa2_fwd_workspace_size(batch, heads_q, heads_kv, seqlen_q, max_kv_len, head_dim);
}

int mi_fa2_fwd_paged(int32_t dtype, const void* q, const void* k_pool, const void* v_pool,
                     void* o, float* lse, const int32_t* block_table, int64_t block_table_stride,
                     const int32_t* kv_lens, int32_t batch, int32_t heads_q, int32_t heads_kv,
                     int32_t seqlen_q, int32_t max_kv_len, int32_t head_dim, int32_t block_size,
                     int32_t num_blocks, const int64_t* q_strides, const int64_t* pool_strides,
                     const int64_t* o_strides, const int64_t* lse_strides, int32_t is_causal,
                     float sm_scale, void* workspace, size_t workspace_bytes,
                     mi_fa2_stream_t stream) {
  return fwd_paged(dtype, q, k_pool, v_pool, o, lse, block_table, block_table_stride, kv_lens,
                   batch, heads_q, heads_kv, seqlen_q, max_kv_len, head_dim, block_size,
                   num_blocks, q_strides, pool_strides, o_strides, lse_strides, is_causal,
                   sm_scale, workspace, workspace_bytes, false, stream);
}

int mi_fa2_fwd_paged_noalloc(int32_t dtype, const void* q, const void* k_pool,
                             const void* v_pool, void* o, float* lse, const int32_t* block_table,
                             int64_t block_table_stride, const int32_t* kv_lens, int32_t batch,
                             int32_t heads_q, int32_t heads_kv, int32_t seqlen_q,
                             int32_t max_kv_len, int32_t head_dim, int32_t block_size,
                             int32_t num_blocks, const int64_t* q_strides,
                             const int64_t* pool_strides, const int64_t* o_strides,
                             const int64_t* lse_strides, int32_t is_causal, float sm_scale,
                             mi_fa2_stream_t stream) {
  return fwd_paged(dtype, q, k_pool, v_pool, o, lse, block_table, block_table_stride, kv_lens,
                   batch, heads_q, heads_kv, seqlen_q, max_kv_len, head_dim, block_size,
                   num_blocks, q_strides, pool_strides, o_strides, lse_strides, is_causal,
                   sm_scale, nullptr, 0, true, stream);
}

int mi_fa2_fwd_paged_varlen(int32_t dtype, const void* q, const void* k_pool, const void* v_pool,
                            void* o, float* lse, const int32_t* cu_seqlens_q,
                            const int32_t* block_table, int64_t block_table_stride,
                            const int32_t* kv_lens, int32_t batch, int32_t heads_q,
                            int32_t heads_kv, int32_t max_seqlen_q, int32_t max_kv_len,
                            int32_t head_dim, int32_t block_size, int32_t num_blocks,
                            const int64_t* q_strides, const int64_t* pool_strides,
                            const int64_t* o_strides, const int64_t* lse_strides,
                            int32_t is_causal, float sm_scale, mi_fa2_stream_t stream) {
  if (int rc = check_common(dtype, batch, heads_q, heads_kv, head_dim)) return rc;
  if (max_seqlen_q < 0 || max_kv_len < 0)
    return fail(MI_FA2_ERR_INVALID, "bad lengths: max_seqlen_q=%d max_kv_len=%d", max_seqlen_q,
                max_kv_len);
  if (block_size < 16 || (block_size & (block_size - 1)))
    return fail(MI_FA2_ERR_UNSUPPORTED, "block_size %d is not a power of two >= 16", block_size);
  if (num_blocks < 0) return fail(MI_FA2_ERR_INVALID, "num_blocks %d < 0", num_blocks);
  if (batch == 0 || max_seqlen_q == 0) return ok();
  if (!cu_seqlens_q) return fail(MI_FA2_ERR_INVALID, "cu_seqlens_q is NULL");
  if (!kv_lens) return fail(MI_FA2_ERR_INVALID, "kv_lens is NULL");
  if (max_kv_len > 0 && !block_table) return fail(MI_FA2_ERR_INVALID, "block_table is NULL");
  if (int rc = check_tensor("q", q, q_strides, 2)) return rc;
  if (int rc = check_tensor("o", o, o_strides, 2)) return rc;
  if (int rc = check_tensor("k_pool", k_pool, pool_strides, 2)) return rc;
  if (int rc = check_tensor("v_pool", v_pool, pool_strides, 2)) return rc;
  if (int rc = check_pitch("pool", pool_strides[0])) return rc;
  if (lse && !lse_strides) return fail(MI_FA2_ERR_INVALID, "lse strides are NULL");

  FwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k_pool);
  p.v = static_cast<const uint16_t*>(v_pool);
  p.o = static_cast<uint16_t*>(o);
  p.cu_q = cu_seqlens_q;
  p.kv_lens = kv_lens;
  p.block_table = block_table;
  p.bt_stride = block_table_stride;
  p.block_size = block_size;
  p.num_blocks = num_blocks;
  p.q_st = q_strides[0], p.q_sh = q_strides[1];
  p.o_st = o_strides[0], p.o_sh = o_strides[1];
  p.k_st = pool_strides[0], p.k_sh = pool_strides[1];
  p.v_st = pool_strides[0], p.v_sh = pool_strides[1];
  set_lse(p, lse, lse_strides, 2);
  p.B = batch;
  p.Hq = heads_q;
  p.Hkv = heads_kv;
  p.group = heads_q / heads_kv;
  p.S = max_kv_len;
  p.causal = is_causal ? 1 : 0;
  p.scale_log2 = sm_scale * mi_fa2::kLog2e;
  if (int rc = check_prefill_strides(p.k_st, p.v_st)) return rc;
  if (int rc = set_device(p)) return rc;
  return launched(mi_fa2::launch_prefill(p, dtype, mi_fa2::kPagedVarlen, max_seqlen_q,
                                         reinterpret_cast<hipStream_t>(stream)));
}

int mi_fa2_combine(int32_t out_dtype, const float* part_o, const float* part_lse,
                   const int32_t* n_parts, int32_t n_rows, int32_t heads, int32_t max_parts,
                   int32_t head_dim, const int64_t* part_o_strides,
                   const int64_t* part_lse_strides, void* o, const int64_t* o_strides, float* lse,
                   const int64_t* lse_strides, mi_fa2_stream_t stream) {
  if (out_dtype != MI_FA2_BF16 && out_dtype != MI_FA2_FP16 && out_dtype != MI_FA2_FP32)
    return fail(MI_FA2_ERR_UNSUPPORTED, "out_dtype %d is not bf16 (0), fp16 (1) or fp32 (2)",
                out_dtype);
  if (head_dim != mi_fa2::kHeadDim)
    return fail(MI_FA2_ERR_UNSUPPORTED, "head_dim %d: the kernel is built for head_dim 128",
                head_dim);
  if (n_rows < 0 || heads < 0 || max_parts < 0 || n_rows > 65535)
    return fail(MI_FA2_ERR_INVALID, "bad sizes: n_rows=%d (at most 65535) heads=%d max_parts=%d",
                n_rows, heads, max_parts);
  if (n_rows == 0 || heads == 0) return ok();
  if (!o || !o_strides) return fail(MI_FA2_ERR_INVALID, "o or its strides are NULL");
  if (lse && !lse_strides) return fail(MI_FA2_ERR_INVALID, "lse strides are NULL");
  if (max_parts > 0 && (!part_o || !part_lse || !part_o_strides || !part_lse_strides))
    return fail(MI_FA2_ERR_INVALID, "partials or their strides are NULL");
  // 8-byte fp32 pairs per lane in, 4 (16-bit) or 8 (fp32) bytes per lane out
  const uintptr_t out_align = out_dtype == MI_FA2_FP32 ? 8 : 4;
  if (reinterpret_cast<uintptr_t>(o) % out_align ||
      (max_parts > 0 && reinterpret_cast<uintptr_t>(part_o) % 8))
    return fail(MI_FA2_ERR_INVALID, "o or part_o is not aligned for its paired stores / loads");
  bool even = o_strides[0] % 2 == 0 && o_strides[1] % 2 == 0;
  for (int i = 0; max_parts > 0 && i < 3; ++i) even = even && part_o_strides[i] % 2 == 0;
  if (!even) return fail(MI_FA2_ERR_INVALID, "o and part_o strides must be even (element pairs)");
  mi_fa2::MergeParams p{};
  p.part_o = part_o;
  p.part_lse = part_lse;
  p.n_parts = n_parts;
  if (max_parts > 0) {
    p.po_sp = part_o_strides[0], p.po_sr = part_o_strides[1], p.po_sh = part_o_strides[2];
    p.pl_sp = part_lse_strides[0], p.pl_sr = part_lse_strides[1], p.pl_sh = part_lse_strides[2];
  }
  p.o = o;
  p.o_sr = o_strides[0], p.o_sh = o_strides[1];
  p.lse = lse;
  if (lse) p.l_sr = lse_strides[0], p.l_sh = lse_strides[1];
  p.rows = n_rows;
  p.heads = heads;
  p.max_parts = max_parts;
  return launched(mi_fa2::launch_merge(p, out_dtype, reinterpret_cast<hipStream_t>(stream)));
}

}  // extern "C"


int mi_fa2_rope_kv_write(int32_t dtype, const void* qkv, int64_t qkv_row_stride, const void* cos,
                         const void* sin, int64_t cs_row_stride, const int32_t* slot_mapping,
                         int32_t n_tokens, int32_t heads_q, int32_t heads_kv, int32_t head_dim,
                         void* q_out, int64_t q_row_stride, void* k_pool, void* v_pool,
                         const int64_t* pool_strides, int32_t num_slots, mi_fa2_stream_t stream) {
  if (dtype != MI_FA2_BF16 && dtype != MI_FA2_FP16)
    return fail(MI_FA2_ERR_UNSUPPORTED, "dtype %d is not bf16 (0) or fp16 (1)", dtype);
  if (head_dim != mi_fa2::kHeadDim)
    return fail(MI_FA2_ERR_UNSUPPORTED, "head_dim %d: the kernel is built for head_dim 128", head_dim);
  if (n_tokens < 0 || heads_q <= 0 || heads_kv <= 0 || num_slots < 0)
    return fail(MI_FA2_ERR_INVALID, "bad sizes: n_tokens=%d heads_q=%d heads_kv=%d num_slots=%d",
                n_tokens, heads_q, heads_kv, num_slots);
  if (n_tokens == 0) return ok();
  const void* ptrs[] = {qkv, cos, sin, q_out, k_pool, v_pool};
  const char* names[] = {"qkv", "cos", "sin", "q_out", "k_pool", "v_pool"};
  for (int i = 0; i < 6; ++i) {
    if (!ptrs[i]) return fail(MI_FA2_ERR_INVALID, "%s is NULL", names[i]);
    if (!aligned16(ptrs[i])) return fail(MI_FA2_ERR_INVALID, "%s is not 16-byte aligned", names[i]);
  }
  if (!slot_mapping) return fail(MI_FA2_ERR_INVALID, "slot_mapping is NULL");
  if (!pool_strides) return fail(MI_FA2_ERR_INVALID, "pool strides are NULL");
  const int64_t strides[] = {qkv_row_stride, cs_row_stride, q_row_stride, pool_strides[0],
                             pool_strides[1]};
  for (int64_t st : strides)
    if (st <= 0 || st % 8)
      return fail(MI_FA2_ERR_INVALID, "stride %lld is not a positive multiple of 8 elements",
                  (long long)st);
  if (qkv_row_stride < (int64_t)(heads_q + 2 * heads_kv) * mi_fa2::kHeadDim ||
      cs_row_stride < mi_fa2::kHeadDim || q_row_stride < (int64_t)heads_q * mi_fa2::kHeadDim)
    return fail(MI_FA2_ERR_INVALID, "row strides shorter than a row");
  mi_fa2::RopeParams p{};
  p.qkv = static_cast<const uint16_t*>(qkv);
  p.qkv_st = qkv_row_stride;
  p.cos = static_cast<const uint16_t*>(cos);
  p.sin = static_cast<const uint16_t*>(sin);
  p.cs_st = cs_row_stride;
  p.slots = slot_mapping;
  p.q_out = static_cast<uint16_t*>(q_out);
  p.q_st = q_row_stride;
  p.k_pool = static_cast<uint16_t*>(k_pool);
  p.v_pool = static_cast<uint16_t*>(v_pool);
  p.pool_st = pool_strides[0];
  p.pool_sh = pool_strides[1];
  p.num_slots = num_slots;
  p.n_tokens = n_tokens;
  p.Hq = heads_q;
  p.Hkv = heads_kv;
  return launched(mi_fa2::launch_rope_kv(p, dtype, reinterpret_cast<hipStream_t>(stream)));
}

size_t mi_fa2_sample_workspace_size(int32_t batch, int32_t vocab) {
  if (batch <= 0 || vocab <= 0) return 0;
  const int chunks = mi_fa2::sample_chunks(vocab);
  return chunks > 1 ? (size_t)batch * chunks * (sizeof(float) + sizeof(int32_t)) : 0;
}

int mi_fa2_sample(int32_t dtype, const void* logits, int64_t row_stride, int32_t batch,
                  int32_t vocab, float temperature, uint64_t seed, uint64_t offset, int32_t* tokens,
                  void* workspace, size_t workspace_bytes, mi_fa2_stream_t stream) {
  if (dtype != MI_FA2_BF16 && dtype != MI_FA2_FP16 && dtype != MI_FA2_FP32)
    return fail(MI_FA2_ERR_UNSUPPORTED, "dtype %d is not bf16 (0), fp16 (1) or fp32 (2)", dtype);
  if (batch < 0 || vocab <= 0 || vocab > (1 << 30))
    return fail(MI_FA2_ERR_INVALID, "bad sizes: batch=%d vocab=%d", batch, vocab);
  if (batch > 65535)
    return fail(MI_FA2_ERR_UNSUPPORTED, "batch %d exceeds 65535 rows per call", batch);
  if (temperature != temperature) return fail(MI_FA2_ERR_INVALID, "temperature is NaN");
  if (batch == 0) return ok();
  if (!logits) return fail(MI_FA2_ERR_INVALID, "logits is NULL");
  if (!tokens) return fail(MI_FA2_ERR_INVALID, "tokens is NULL");
  const uintptr_t elem = dtype == MI_FA2_FP32 ? 4 : 2;
  if (reinterpret_cast<uintptr_t>(logits) % elem)
    return fail(MI_FA2_ERR_INVALID, "logits is not aligned to its element size");
  if (row_stride < vocab)
    return fail(MI_FA2_ERR_INVALID, "row_stride %lld is shorter than a row of %d",
                (long long)row_stride, vocab);
  const size_t need = mi_fa2_sample_workspace_size(batch, vocab);
  if (need && (!workspace || workspace_bytes < need))
    return fail(MI_FA2_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need,
                workspace ? workspace_bytes : (size_t)0);
  mi_fa2::SampleParams p{};
  p.logits = logits;
  p.row_stride = row_stride;
  p.tokens = tokens;
  p.batch = batch;
  p.vocab = vocab;
  p.chunks = mi_fa2::sample_chunks(vocab);
  p.greedy = temperature > 0.f ? 0 : 1;
  p.inv_t = temperature > 0.f ? 1.f / temperature : 0.f;
  p.seed_lo = (uint32_t)seed;
  p.seed_hi = (uint32_t)(seed >> 32);
  p.off_lo = (uint32_t)offset;
  p.off_hi = (uint32_t)(offset >> 32);
  if (need) {
    p.part_s = static_cast<float*>(workspace);
    p.part_i = reinterpret_cast<int32_t*>(p.part_s + (size_t)batch * p.chunks);
  }
  return launched(mi_fa2::launch_sample(p, dtype, reinterpret_cast<hipStream_t>(stream)));
}

int mi_fa2_step_metadata(const int32_t* row_slots, const int32_t* cu, int32_t tokens_per_row,
                         int32_t batch, int32_t* seq_lens, int32_t max_seqs, const int32_t* tables,
                         int64_t table_stride, int32_t block_size, int32_t width, int32_t* starts,
                         int32_t* kv_lens, int32_t* block_table, int32_t* slots,
                         int32_t* positions, int32_t* last_idx, mi_fa2_stream_t stream) {
  if (batch < 0 || max_seqs <= 0 || table_stride <= 0 || block_size <= 0 || width <= 0 ||
      (!cu && tokens_per_row < 0))
    return fail(MI_FA2_ERR_INVALID,
                "bad sizes: batch=%d max_seqs=%d table_stride=%lld block_size=%d width=%d "
                "tokens_per_row=%d", batch, max_seqs, (long long)table_stride, block_size, width,
                tokens_per_row);
  if (batch == 0) return ok();
  const void* ptrs[] = {row_slots, seq_lens, tables, starts, kv_lens, block_table, slots};
  const char* names[] = {"row_slots", "seq_lens", "tables", "starts", "kv_lens", "block_table",
                         "slots"};
  for (int i = 0; i < 7; ++i)
    if (!ptrs[i]) return fail(MI_FA2_ERR_INVALID, "%s is NULL", names[i]);
  mi_fa2::StepMetaParams p{};
  p.row_slots = row_slots;
  p.cu = cu;
  p.T = tokens_per_row;
  p.B = batch;
  p.W = width;
  p.block_size = block_size;
  p.max_seqs = max_seqs;
  p.seq_lens = seq_lens;
  p.tables = tables;
  p.table_stride = table_stride;
  p.starts = starts;
  p.kv_lens = kv_lens;
  p.block_table = block_table;
  p.slots = slots;
  p.positions = positions;
  p.last_idx = last_idx;
  return launched(mi_fa2::launch_step_meta(p, reinterpret_cast<hipStream_t>(stream)));
}

namespace {
int check_rows(const char* name, const void* ptr, int64_t stride, int64_t min_stride) {
  if (!ptr) return fail(MI_FA2_ERR_INVALID, "%s is NULL", name);
  if (!aligned16(ptr)) return fail(MI_FA2_ERR_INVALID, "%s is not 16-byte aligned", name);
  if (stride < min_stride || stride % 8)
    return fail(MI_FA2_ERR_INVALID, "%s row stride %lld: a multiple of 8 of at least %lld needed",
                name, (long long)stride, (long long)min_stride);
  return MI_FA2_OK;
}
}  // namespace

int mi_fa2_add_rmsnorm(int32_t dtype, const void* x, int64_t x_stride, const void* y,
                       int64_t y_stride, const void* weight, void* residual_out,
                       int64_t residual_stride, void* out, int64_t out_stride, int32_t rows,
                       int32_t hidden, float eps, mi_fa2_stream_t stream) {
  if (dtype != MI_FA2_BF16 && dtype != MI_FA2_FP16)
    return fail(MI_FA2_ERR_UNSUPPORTED, "dtype %d is not bf16 (0) or fp16 (1)", dtype);
  if (rows < 0 || hidden <= 0 || hidden % 8 || hidden > 8192)
    return fail(MI_FA2_ERR_INVALID, "bad sizes: rows=%d hidden=%d (hidden: a multiple of 8, <= 8192)",
                rows, hidden);
  if (rows == 0) return ok();
  if (int rc = check_rows("x", x, x_stride, hidden)) return rc;
  if (y)
    if (int rc = check_rows("y", y, y_stride, hidden)) return rc;
  if (residual_out)
    if (int rc = check_rows("residual_out", residual_out, residual_stride, hidden)) return rc;
  if (int rc = check_rows("out", out, out_stride, hidden)) return rc;
  if (!weight || !aligned16(weight))
    return fail(MI_FA2_ERR_INVALID, "weight is NULL or not 16-byte aligned");
  mi_fa2::ModelOpParams p{};
  p.x = static_cast<const uint16_t*>(x);
  p.x_st = x_stride;
  p.y = static_cast<const uint16_t*>(y);
  p.y_st = y_stride;
  p.weight = static_cast<const uint16_t*>(weight);
  p.r_out = y ? static_cast<uint16_t*>(residual_out) : nullptr;
  p.r_st = residual_stride;
  p.out = static_cast<uint16_t*>(out);
  p.out_st = out_stride;
  p.rows = rows;
  p.hidden = hidden;
  p.eps = eps;
  return launched(mi_fa2::launch_add_rmsnorm(p, dtype, reinterpret_cast<hipStream_t>(stream)));
}

int mi_fa2_silu_mul(int32_t dtype, const void* gate_up, int64_t gate_up_stride, void* out,
                    int64_t out_stride, int32_t rows, int32_t inter, mi_fa2_stream_t stream) {
  if (dtype != MI_FA2_BF16 && dtype != MI_FA2_FP16)
    return fail(MI_FA2_ERR_UNSUPPORTED, "dtype %d is not bf16 (0) or fp16 (1)", dtype);
  if (rows < 0 || inter <= 0 || inter % 8)
    return fail(MI_FA2_ERR_INVALID, "bad sizes: rows=%d inter=%d (a multiple of 8)", rows, inter);
  if (rows == 0) return ok();
  if (int rc = check_rows("gate_up", gate_up, gate_up_stride, 2 * (int64_t)inter)) return rc;
  if (int rc = check_rows("out", out, out_stride, inter)) return rc;
  mi_fa2::ModelOpParams p{};
  p.x = static_cast<const uint16_t*>(gate_up);
  p.x_st = gate_up_stride;
  p.out = static_cast<uint16_t*>(out);
  p.out_st = out_stride;
  p.rows = rows;
  p.hidden = inter;
  return launched(mi_fa2::launch_silu_mul(p, dtype, reinterpret_cast<hipStream_t>(stream)));
}
