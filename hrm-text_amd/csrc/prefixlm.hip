// C ABI of the gfx950 PrefixLM attention library (declared in include/prefixlm.h).
//
// Host-side validation, workspace carving and kernel launches. The library keeps
// no state between calls except (a) a thread-local error string and (b) a one-time
// per-process kernel attribute setup; timing records live in caller-owned timers.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>
#include <new>
#include <vector>

#include "prefixlm.h"
#include "common.h"
#include "worklist.h"
#include "fwd.h"
#include "bwd.h"
#include "plan.h"
#include "rope.h"
#include "kvcache.h"
#include "norm_mlp.h"
#include "gemm.h"

using namespace prefixlm;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Stored dS of the dQ-from-dS backward: per head, one 4 KB block (32 queries x 64 keys)
// per attended (key group, query tile) of every segment, in the layout of ds_blk_off
// (worklist.h), from ds_base[s] on. The host scalars bound the blocks per head by
// sum_s ceil(L_s / 32) * ceil(L_s / 64) <= (num_tokens / 32 + numseqs + 1) *
// ceil(max_seqlen_all / 64); a plan knows the exact count. Scales: one per 128-key tile,
// slot (cu_seqlens[s] + k) / 128 + s, below num_tokens / 128 + numseqs + 1.
int64_t ds_bound_blocks(int32_t T, int32_t numseqs, int32_t max_all) {
  return ((int64_t)T / 32 + numseqs + 1) * (((int64_t)max_all + 63) / 64);
}
int64_t ds_nkslot(int32_t T, int32_t numseqs) { return (int64_t)T / 128 + numseqs + 1; }

int64_t max_items(int32_t total, int32_t numseqs, int tile) {
  return (int64_t)(total + tile - 1) / tile + numseqs;
}

// The three lists of a host plan, in the order and with the parameters of the
// device-built lists (forward; backward dK/dV; backward dQ).
const plan::ListDesc kPlanLists[plan::kLists] = {
    {0, fwd::BM, fwd::BN}, {1, bwd::kv::BK, bwd::kv::BQ}, {0, bwd::qk::BQ, bwd::qk::BKT}};

// Checks a caller's plan against this call's scalars; returns its layout.
int check_plan(const void* p, size_t bytes, int32_t total, int32_t numseqs, plan::Layout* l) {
  *l = plan::layout(kPlanLists, total, numseqs);
  if (!p) return fail(PREFIXLM_ERR_INVALID, "plan pointer is null");
  if ((reinterpret_cast<uintptr_t>(p) & 255u) != 0)
    return fail(PREFIXLM_ERR_INVALID, "plan must be 256-byte aligned");
  if (bytes != l->bytes)
    return fail(PREFIXLM_ERR_INVALID,
                "plan of %zu bytes, a batch with total_seqlen=%d and numseqs=%d has %zu: the plan was "
                "built for other metadata",
                bytes, total, numseqs, l->bytes);
  return PREFIXLM_OK;
}

// ---- optional per-kernel timing ---------------------------------------------------
// Caller-owned: a prefixlm_timer (prefixlm_timer_create) passed in the args collects
// one pair of HIP events around each launch; the library itself keeps no records.
struct TimingRec {
  int id;
  hipEvent_t a, b;
};

}  // namespace

struct prefixlm_timer {
  std::vector<TimingRec> recs;
  std::vector<hipEvent_t> pool;
  hipEvent_t get() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
};

namespace {

struct KernelTimer {
  prefixlm_timer* t;
  int id;
  hipStream_t s;
  hipEvent_t a = nullptr, b = nullptr;
  KernelTimer(void* timer, int id_, hipStream_t s_) : t(static_cast<prefixlm_timer*>(timer)), id(id_), s(s_) {
    if (!t) return;
    a = t->get();
    b = t->get();
    if (a && b && hipEventRecord(a, s) != hipSuccess) a = b = nullptr;
  }
  ~KernelTimer() {
    if (!(a && b)) return;
    if (hipEventRecord(b, s) == hipSuccess) t->recs.push_back({id, a, b});
  }
};

std::once_flag g_attr_once;
hipError_t g_attr_err = hipSuccess;
void set_kernel_attrs() {
  std::call_once(g_attr_once, [] {
    g_attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&fwd::prefixlm_fwd_kernel<128>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, fwd::Geo<128>::LDS_BYTES);
    if (g_attr_err == hipSuccess)
      g_attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&fwd::prefixlm_fwd_kernel<64>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, fwd::Geo<64>::LDS_BYTES);
    if (g_attr_err == hipSuccess)
      g_attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&bwd::prefixlm_bwd_dkdv_kernel<128>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bwd::kv::Geo<128>::LDS_BYTES);
    if (g_attr_err == hipSuccess)
      g_attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&bwd::prefixlm_bwd_dkdv_kernel<64>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bwd::kv::Geo<64>::LDS_BYTES);
    if (g_attr_err == hipSuccess)
      g_attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&bwd::prefixlm_bwd_dq_kernel<128>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bwd::qk::Geo<128>::LDS_BYTES);
    if (g_attr_err == hipSuccess)
      g_attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&bwd::prefixlm_bwd_dq_kernel<64>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bwd::qk::Geo<64>::LDS_BYTES);
    if (g_attr_err == hipSuccess)
      g_attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&bwd::prefixlm_bwd_dq_ds_kernel<128>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bwd::q2::Geo<128>::LDS_BYTES);
    if (g_attr_err == hipSuccess)
      g_attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&bwd::prefixlm_bwd_dq_ds_kernel<64>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bwd::q2::Geo<64>::LDS_BYTES);
  });
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Workgroups of a persistent grid with one workgroup per CU: the current device's CU
// count rounded down to a multiple of 8 (the XCD count; the kernels take work from
// per-XCD counters). Cached per device.
std::mutex g_cu_mu;
int g_cu_count[64] = {};
int persistent_grid(int* out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(PREFIXLM_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return fail(PREFIXLM_ERR_INVALID, "device %d >= 64", dev);
  std::lock_guard<std::mutex> g(g_cu_mu);
  if (!g_cu_count[dev]) {
    int n = 0;
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess || n < 1)
      return fail(PREFIXLM_ERR_HIP, "hipDeviceGetAttribute(multiprocessor count): %s", hipGetErrorString(e));
    g_cu_count[dev] = n >= 8 ? n / 8 * 8 : 8;
  }
  *out = g_cu_count[dev];
  return PREFIXLM_OK;
}

// Checks shared by forward and backward. `strides` lists (stride_t, stride_h) pairs.
int check_common(const void* const* ptrs, int nptr, const int64_t* strides, int nstr,
                 int32_t T, int32_t H, int32_t D, int32_t total, int32_t numseqs,
                 int32_t max_all, int64_t meta_len, const int32_t* pre, const int32_t* cau,
                 const int32_t* cu) {
  if (D != 128 && D != 64) return fail(PREFIXLM_ERR_INVALID, "head_dim must be 64 or 128 (got %d)", D);
  if (T < 1 || H < 1) return fail(PREFIXLM_ERR_INVALID, "num_tokens=%d num_heads=%d must be >= 1", T, H);
  if (total < 0 || total > T)
    return fail(PREFIXLM_ERR_INVALID, "total_seqlen=%d outside [0, num_tokens=%d]", total, T);
  if (numseqs < 0) return fail(PREFIXLM_ERR_INVALID, "numseqs=%d < 0", numseqs);
  if (numseqs > 0 && (int64_t)numseqs + 1 > meta_len)
    return fail(PREFIXLM_ERR_INVALID, "numseqs=%d needs %d cu_seqlens entries, arrays hold %lld",
                numseqs, numseqs + 1, (long long)meta_len);
  if (numseqs > 0 && (!pre || !cau || !cu))
    return fail(PREFIXLM_ERR_INVALID, "metadata pointers must be non-null");
  if (max_all < 0 || max_all > total)
    return fail(PREFIXLM_ERR_INVALID, "max_seqlen_all=%d outside [0, total_seqlen=%d]", max_all, total);
  for (int i = 0; i < nptr; ++i) {
    if (!ptrs[i]) return fail(PREFIXLM_ERR_INVALID, "tensor pointer %d is null", i);
    if (!aligned16(ptrs[i]))
      return fail(PREFIXLM_ERR_INVALID, "tensor pointer %d is not 16-byte aligned", i);
  }
  for (int i = 0; i < nstr; ++i) {
    const int64_t st = strides[2 * i], sh = strides[2 * i + 1];
    if (st < D || sh < 0 || (st % 8) != 0 || (sh % 8) != 0)
      return fail(PREFIXLM_ERR_INVALID,
                  "tensor %d strides (token %lld, head %lld) must be multiples of 8 with token "
                  "stride >= head_dim and head stride >= 0",
                  i, (long long)st, (long long)sh);
    // buffer offsets inside one segment are 32-bit byte offsets
    if (((int64_t)max_all + 256) * st * 2 >= (int64_t)1 << 31)
      return fail(PREFIXLM_ERR_INVALID, "segment of %d rows x token stride %lld exceeds 2 GiB",
                  max_all, (long long)st);
  }
  return PREFIXLM_OK;
}

}  // namespace

// ---- scratch of the zero-allocation backward ------------------------------------
// Device memory of prefixlm_bwd_noalloc: a file-scope array each GPU holds (at its own
// address) from the library's load until the process ends. Its host-side name is not a
// device address: kernels only ever receive the address hipGetSymbolAddress returns,
// fetched once per device with that device current.
constexpr size_t kNoallocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Address of this device's scratch array (the current device's).
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(PREFIXLM_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(PREFIXLM_ERR_INVALID, "device %d >= %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(PREFIXLM_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PREFIXLM_OK;
}
}  // namespace

extern "C" {

int32_t prefixlm_version(void) { return PREFIXLM_VERSION; }

const char* prefixlm_last_error(void) { return g_err; }

size_t prefixlm_fwd_workspace_size(int32_t num_tokens, int32_t num_heads, int32_t head_dim,
                                   int32_t total_seqlen, int32_t numseqs) {
  // the work list (either head dim runs its own kernel)
  (void)num_tokens;
  (void)num_heads;
  (void)head_dim;
  return align_up(sizeof(WsHeader)) + align_up(sizeof(int2) * (size_t)max_items(total_seqlen, numseqs, fwd::BM));
}

size_t prefixlm_fwd_q_amax_count(int32_t num_tokens, int32_t num_heads) {
  // a slot per wave of the forward grid, for any numseqs <= num_tokens
  if (num_tokens < 0 || num_heads < 1) return 0;
  return (size_t)(fwd::NT / 64) * unit_grid(max_items(num_tokens, num_tokens, fwd::BM), num_heads);
}

size_t prefixlm_bwd_workspace_size(int32_t num_tokens, int32_t num_heads, int32_t head_dim,
                                   int32_t total_seqlen, int32_t numseqs) {
  // the same for either head dim: work lists (the dK/dV list's header, which carries the
  // error word, first), stored-dS bases, statistics, counters and delta
  (void)head_dim;
  return align_up(sizeof(WsHeader)) +                                                   // dK/dV list
         align_up(sizeof(int2) * (size_t)max_items(total_seqlen, numseqs, bwd::kv::BK)) +
         align_up(sizeof(WsHeader)) +                                                   // dQ list
         align_up(sizeof(int2) * (size_t)max_items(total_seqlen, numseqs, bwd::qk::BQ)) +
         align_up(sizeof(int32_t) * ((size_t)numseqs + 1)) +                            // dS bases
         align_up(sizeof(float) * ((size_t)num_heads * bwd::kStats +                    // statistics
                                   (size_t)numseqs * num_heads * bwd::kSegStats + bwd::kCounters)) +
         align_up(sizeof(float) * (size_t)num_heads * num_tokens);                      // delta
}

size_t prefixlm_bwd_ds_bytes_blocks(int32_t num_tokens, int32_t num_heads, int32_t numseqs, int64_t ds_blocks) {
  if (num_tokens < 1 || num_heads < 1 || numseqs < 0 || ds_blocks < 1) return 0;
  const int64_t hb = ds_blocks * 4096;
  if (hb >= ((int64_t)1 << 31)) return 0;   // one head's blocks must fit 32-bit offsets
  return align_up((size_t)hb * num_heads) + align_up(sizeof(float) * (size_t)num_heads * ds_nkslot(num_tokens, numseqs));
}

size_t prefixlm_bwd_ds_bytes(int32_t num_tokens, int32_t num_heads, int32_t numseqs, int32_t max_seqlen_all) {
  if (max_seqlen_all < 1 || max_seqlen_all > 128 * bwd::q2::MAX_KT) return 0;   // the dQ kernel holds a segment's tile scales in LDS
  return prefixlm_bwd_ds_bytes_blocks(num_tokens, num_heads, numseqs, ds_bound_blocks(num_tokens, numseqs, max_seqlen_all));
}

}  // extern "C"

template <int HD>
static int fwd_launch(const prefixlm_fwd_args* a, void* stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (a->struct_size != sizeof(prefixlm_fwd_args))
    return fail(PREFIXLM_ERR_INVALID, "prefixlm_fwd_args.struct_size is %u, this library's is %zu: the caller was "
                "built against another version of prefixlm.h", a->struct_size, sizeof(prefixlm_fwd_args));
  const int has_lo = a->out_lo != nullptr;
  const bool use_plan = a->plan != nullptr;
  const bool gated = a->gate != nullptr;
  if (gated && !has_lo) return fail(PREFIXLM_ERR_INVALID, "a gated forward needs out_lo");
  if (gated && HD != 128) return fail(PREFIXLM_ERR_INVALID, "the output gate needs head_dim 128");
  // with a plan the forward needs no workspace
  const void* ptrs[] = {a->q,       a->k,    a->v, a->out, a->lse, use_plan ? a->q : a->workspace,
                        a->out_lo,  a->gate, a->out_gated};
  const int64_t strides[] = {a->q_stride_t,       a->q_stride_h,       a->k_stride_t,        a->k_stride_h,
                             a->v_stride_t,       a->v_stride_h,       a->out_stride_t,      a->out_stride_h,
                             a->out_lo_stride_t,  a->out_lo_stride_h,  a->gate_stride_t,     a->gate_stride_h,
                             a->out_gated_stride_t, a->out_gated_stride_h};
  int rc = check_common(ptrs, 6 + has_lo + 2 * gated, strides, 4 + has_lo + 2 * gated, a->num_tokens,
                        a->num_heads, a->head_dim, a->total_seqlen, a->numseqs, a->max_seqlen_all, a->meta_len,
                        a->prefix_lens, a->causal_lens, a->cu_seqlens);
  if (rc) return rc;
  // out_lo rows (int8, head_dim bytes) leave the kernel as 16-byte chunks
  if (has_lo && ((a->out_lo_stride_t % 16) != 0 || (a->out_lo_stride_h % 16) != 0))
    return fail(PREFIXLM_ERR_INVALID, "out_lo strides (token %lld, head %lld) must be multiples of 16",
                (long long)a->out_lo_stride_t, (long long)a->out_lo_stride_h);
  plan::Layout pl{};
  if (use_plan) {
    rc = check_plan(a->plan, a->plan_bytes, a->total_seqlen, a->numseqs, &pl);
    if (rc) return rc;
  } else {
    const size_t need = prefixlm_fwd_workspace_size(a->num_tokens, a->num_heads, HD, a->total_seqlen, a->numseqs);
    if (a->workspace_bytes < need)
      return fail(PREFIXLM_ERR_INVALID, "workspace of %zu bytes, %zu needed", a->workspace_bytes, need);
  }
  if (a->q_amax != nullptr && a->numseqs > a->num_tokens)
    return fail(PREFIXLM_ERR_INVALID, "q_amax holds prefixlm_fwd_q_amax_count(num_tokens, num_heads) slots, "
                "which assumes numseqs <= num_tokens (got numseqs=%d, num_tokens=%d)", a->numseqs, a->num_tokens);
  set_kernel_attrs();
  if (g_attr_err != hipSuccess)
    return fail(PREFIXLM_ERR_HIP, "hipFuncSetAttribute: %s", hipGetErrorString(g_attr_err));

  const char* lists = use_plan ? static_cast<const char*>(a->plan) : static_cast<const char*>(a->workspace);
  WsHeader* hdr = reinterpret_cast<WsHeader*>(const_cast<char*>(lists) + (use_plan ? pl.hdr_off[0] : 0));
  int2* items = reinterpret_cast<int2*>(const_cast<char*>(lists) +
                                        (use_plan ? pl.items_off[0] : align_up(sizeof(WsHeader))));
  const int64_t nmax = max_items(a->total_seqlen, a->numseqs, fwd::BM);
  const int T = a->num_tokens, H = a->num_heads;

  (void)hipGetLastError();
  if (!use_plan) {
    // always run, so the workspace header (item count, error word) is fresh
    MetaParams m{a->prefix_lens, a->causal_lens, a->cu_seqlens, a->numseqs, a->total_seqlen, T,
                 a->is_causal ? 1 : 0, a->max_seqlen_all};
    KernelTimer tm(a->timer, 0, stream);
    ListSpecs specs{};
    specs.l[0] = ListSpec{0, fwd::BM, fwd::BN, (int)nmax, items, hdr, nullptr, 0};
    hipLaunchKernelGGL(build_worklist_kernel, dim3(1), dim3(kPrepThreads), 0, stream, m, specs,
                       (float*)nullptr, 0);
  }
  if (nmax > 0) {
    fwd::Params P;
    P.q = static_cast<const bf16*>(a->q);
    P.k = static_cast<const bf16*>(a->k);
    P.v = static_cast<const bf16*>(a->v);
    P.o = static_cast<bf16*>(a->out);
    P.o_lo = static_cast<int8_t*>(a->out_lo);
    P.lse = a->lse;
    P.gate = static_cast<const bf16*>(a->gate);
    P.y = static_cast<bf16*>(a->out_gated);
    P.q_st = a->q_stride_t; P.q_sh = a->q_stride_h;
    P.k_st = a->k_stride_t; P.k_sh = a->k_stride_h;
    P.v_st = a->v_stride_t; P.v_sh = a->v_stride_h;
    P.o_st = a->out_stride_t; P.o_sh = a->out_stride_h;
    P.lo_st = a->out_lo_stride_t; P.lo_sh = a->out_lo_stride_h;
    P.g_st = a->gate_stride_t; P.g_sh = a->gate_stride_h;
    P.y_st = a->out_gated_stride_t; P.y_sh = a->out_gated_stride_h;
    P.prefix = a->prefix_lens;
    P.causal = a->causal_lens;
    P.cu = a->cu_seqlens;
    P.items = items;
    P.hdr = hdr;
    P.q_amax = a->q_amax;
    P.T = T;
    P.H = H;
    P.is_causal = a->is_causal ? 1 : 0;
    P.numseqs = a->numseqs;
    P.scale_log2 = a->softmax_scale * kLog2e;
    const int64_t nblk = unit_grid(nmax, H);
    if (nblk > 0x7fffffff) return fail(PREFIXLM_ERR_INVALID, "grid of %lld blocks too large", (long long)nblk);
    {
      KernelTimer tm(a->timer, 1, stream);
      hipLaunchKernelGGL(fwd::prefixlm_fwd_kernel<HD>, dim3((unsigned)nblk), dim3(fwd::NT),
                         fwd::Geo<HD>::LDS_BYTES, stream, P);
    }
  }
  if (a->total_seqlen < T) {
    const int64_t rows = (int64_t)(T - a->total_seqlen) * H;
    KernelTimer tm(a->timer, 2, stream);
    constexpr int groups = 256 / (HD / 8);   // (row, head) pairs per workgroup
    hipLaunchKernelGGL(fwd::prefixlm_fwd_pad_kernel<HD>, dim3((unsigned)((rows + groups - 1) / groups)), dim3(256), 0,
                       stream, static_cast<bf16*>(a->out), static_cast<int8_t*>(a->out_lo),
                       static_cast<bf16*>(gated ? a->out_gated : nullptr), a->lse, a->out_stride_t,
                       a->out_stride_h, a->out_lo_stride_t, a->out_lo_stride_h, a->out_gated_stride_t,
                       a->out_gated_stride_h, T, H, a->total_seqlen);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PREFIXLM_ERR_HIP, "forward launch: %s", hipGetErrorString(e));
  return PREFIXLM_OK;
}

template <int HD>
static int bwd_launch(const prefixlm_bwd_args* a, void* stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (a->struct_size != sizeof(prefixlm_bwd_args))
    return fail(PREFIXLM_ERR_INVALID, "prefixlm_bwd_args.struct_size is %u, this library's is %zu: the caller was "
                "built against another version of prefixlm.h", a->struct_size, sizeof(prefixlm_bwd_args));
  const void* ptrs[] = {a->q,  a->k,  a->v,  a->out,       a->dout, a->lse,
                        a->dq, a->dk, a->dv, a->workspace, a->out_lo};
  const int64_t strides[] = {a->q_stride_t,    a->q_stride_h,    a->k_stride_t,    a->k_stride_h,
                             a->v_stride_t,    a->v_stride_h,    a->out_stride_t,  a->out_stride_h,
                             a->dout_stride_t, a->dout_stride_h, a->dq_stride_t,   a->dq_stride_h,
                             a->dk_stride_t,   a->dk_stride_h,   a->dv_stride_t,   a->dv_stride_h,
                             a->out_lo_stride_t, a->out_lo_stride_h};
  const int has_lo = a->out_lo != nullptr;
  int rc = check_common(ptrs, 10 + has_lo, strides, 8 + has_lo, a->num_tokens, a->num_heads, a->head_dim,
                        a->total_seqlen, a->numseqs, a->max_seqlen_all, a->meta_len,
                        a->prefix_lens, a->causal_lens, a->cu_seqlens);
  if (rc) return rc;
  const bool gated = a->gate != nullptr;
  if (gated && HD != 128) return fail(PREFIXLM_ERR_INVALID, "the output gate needs head_dim 128");
  if (gated) {
    const void* gp[] = {a->gate, a->dgate, a->dout_attn};
    const int64_t gs[] = {a->gate_stride_t,  a->gate_stride_h,      a->dgate_stride_t,
                          a->dgate_stride_h, a->dout_attn_stride_t, a->dout_attn_stride_h};
    rc = check_common(gp, 3, gs, 3, a->num_tokens, a->num_heads, a->head_dim, a->total_seqlen, a->numseqs,
                      a->max_seqlen_all, a->meta_len, a->prefix_lens, a->causal_lens, a->cu_seqlens);
    if (rc) return rc;
  }
  const bool use_plan = a->plan != nullptr;
  plan::Layout pl{};
  if (use_plan) {
    rc = check_plan(a->plan, a->plan_bytes, a->total_seqlen, a->numseqs, &pl);
    if (rc) return rc;
  }
  const size_t need =
      prefixlm_bwd_workspace_size(a->num_tokens, a->num_heads, HD, a->total_seqlen, a->numseqs);
  if (a->workspace_bytes < need)
    return fail(PREFIXLM_ERR_INVALID, "workspace of %zu bytes, %zu needed", a->workspace_bytes, need);
  // dQ from the stored dS when the caller gave a buffer and the layout fits: a->ds_blocks
  // blocks per head, or the bound the scalars give
  if (a->ds_blocks < 0) return fail(PREFIXLM_ERR_INVALID, "ds_blocks=%lld < 0", (long long)a->ds_blocks);
  const int64_t ds_cap =
      a->ds_blocks > 0 ? a->ds_blocks : ds_bound_blocks(a->num_tokens, a->numseqs, a->max_seqlen_all);
  const size_t ds_need = a->max_seqlen_all > 128 * bwd::q2::MAX_KT
                             ? 0
                             : prefixlm_bwd_ds_bytes_blocks(a->num_tokens, a->num_heads, a->numseqs, ds_cap);
  const bool use_ds = a->ds_buf != nullptr && ds_need > 0;
  if (use_ds) {
    if (a->ds_buf_bytes < ds_need)
      return fail(PREFIXLM_ERR_INVALID, "ds_buf of %zu bytes, %zu needed", a->ds_buf_bytes, ds_need);
    if ((reinterpret_cast<uintptr_t>(a->ds_buf) & 255u) != 0)
      return fail(PREFIXLM_ERR_INVALID, "ds_buf must be 256-byte aligned");
  }
  if (a->num_heads > bwd::kPreMaxHeads)
    return fail(PREFIXLM_ERR_INVALID, "num_heads=%d exceeds %d", a->num_heads, bwd::kPreMaxHeads);
  if (a->q_amax == nullptr)
    return fail(PREFIXLM_ERR_INVALID, "q_amax is null: the backward needs the forward's per-workgroup max |Q| "
                "(prefixlm_fwd_args.q_amax)");
  {
    // the pre-pass addresses kPreRows rows x all heads of out, out_lo and dout with
    // 32-bit byte offsets
    const int64_t st[6] = {a->out_stride_t, a->out_lo_stride_t, a->dout_stride_t,
                           a->gate_stride_t, a->dgate_stride_t, a->dout_attn_stride_t};
    const int64_t sh[6] = {a->out_stride_h, a->out_lo_stride_h, a->dout_stride_h,
                           a->gate_stride_h, a->dgate_stride_h, a->dout_attn_stride_h};
    for (int i = 0; i < 6; ++i) {
      if ((i == 1 && !has_lo) || (i >= 3 && !gated)) continue;
      if (((int64_t)bwd::kPreRows * st[i] + (int64_t)(a->num_heads - 1) * sh[i] + a->head_dim) * 2 >=
          (int64_t)1 << 31)
        return fail(PREFIXLM_ERR_INVALID, "tensor %d spans more than 2 GiB over %d rows", i, bwd::kPreRows);
    }
  }
  set_kernel_attrs();
  if (g_attr_err != hipSuccess)
    return fail(PREFIXLM_ERR_HIP, "hipFuncSetAttribute: %s", hipGetErrorString(g_attr_err));

  const int T = a->num_tokens, H = a->num_heads;
  const int64_t nkv = max_items(a->total_seqlen, a->numseqs, bwd::kv::BK);
  const int64_t nq = max_items(a->total_seqlen, a->numseqs, bwd::qk::BQ);
  if (unit_grid(nkv, H) > 0x7fffffff || unit_grid(nq, H) > 0x7fffffff)
    return fail(PREFIXLM_ERR_INVALID, "grid of %lld blocks too large", (long long)unit_grid(nq, H));
  char* ws = static_cast<char*>(a->workspace);
  size_t off = 0;
  WsHeader* hdr_kv = reinterpret_cast<WsHeader*>(ws + off);
  off += align_up(sizeof(WsHeader));
  int2* items_kv = reinterpret_cast<int2*>(ws + off);
  off += align_up(sizeof(int2) * (size_t)nkv);
  WsHeader* hdr_q = reinterpret_cast<WsHeader*>(ws + off);
  off += align_up(sizeof(WsHeader));
  int2* items_q = reinterpret_cast<int2*>(ws + off);
  off += align_up(sizeof(int2) * (size_t)nq);
  int32_t* ds_base = reinterpret_cast<int32_t*>(ws + off);
  off += align_up(sizeof(int32_t) * ((size_t)a->numseqs + 1));
  float* stats = reinterpret_cast<float*>(ws + off);
  float* segstats = stats + (size_t)H * bwd::kStats;
  // statistics, then the work-item counters of the persistent kernels (all zeroed below)
  const size_t n_stats = (size_t)H * bwd::kStats + (size_t)a->numseqs * H * bwd::kSegStats + bwd::kCounters;
  int* counters = reinterpret_cast<int*>(segstats + (size_t)a->numseqs * H * bwd::kSegStats);
  off += align_up(sizeof(float) * n_stats);
  float* delta = reinterpret_cast<float*>(ws + off);
  if (n_stats > 0x7fffffff) return fail(PREFIXLM_ERR_INVALID, "too many segments");
  if (use_plan) {
    char* pb = static_cast<char*>(const_cast<void*>(a->plan));
    hdr_kv = reinterpret_cast<WsHeader*>(pb + pl.hdr_off[1]);
    items_kv = reinterpret_cast<int2*>(pb + pl.items_off[1]);
    hdr_q = reinterpret_cast<WsHeader*>(pb + pl.hdr_off[2]);
    items_q = reinterpret_cast<int2*>(pb + pl.items_off[2]);
    ds_base = reinterpret_cast<int32_t*>(pb + pl.ds_off);
  }

  (void)hipGetLastError();
  // the forward's max |Q| slots (its grid: one per workgroup), reduced per head by the
  // pre-pass into statistics slot 3, for the dK/dV kernel's fp16 scale of Q
  const int q_slots = (fwd::NT / 64) * (int)unit_grid(max_items(a->total_seqlen, a->numseqs, fwd::BM), H);
  if (use_plan) {
    // the work-list kernel is skipped; clear the statistics it would have cleared
    KernelTimer tm(a->timer, 3, stream);
    const int nb = (int)std::min<size_t>((n_stats + 255) / 256, 1024);
    if (nb > 0)
      hipLaunchKernelGGL(bwd::zero_floats_kernel, dim3(nb), dim3(256), 0, stream, stats, (int)n_stats);
  } else {
    // both work lists; also zeroes the statistics the next kernels accumulate
    MetaParams m{a->prefix_lens, a->causal_lens, a->cu_seqlens, a->numseqs, a->total_seqlen, T,
                 a->is_causal ? 1 : 0, a->max_seqlen_all};
    ListSpecs specs{};
    specs.l[0] = ListSpec{1, bwd::kv::BK, bwd::kv::BQ, (int)nkv, items_kv, hdr_kv, use_ds ? ds_base : nullptr,
                          (int)std::min<int64_t>(ds_cap, 0x7fffffff)};
    specs.l[1] = ListSpec{0, bwd::qk::BQ, bwd::qk::BKT, (int)nq, items_q, hdr_q, nullptr, 0};
    KernelTimer tm(a->timer, 3, stream);
    hipLaunchKernelGGL(build_worklist_kernel, dim3(2), dim3(kPrepThreads), 0, stream, m, specs, stats,
                       (int)n_stats);
  }
  // the dK/dV and dQ kernels read dO: the caller's dout, or with a gate the
  // pre-pass's dout * sigmoid(gate)
  const bf16* dO = static_cast<const bf16*>(gated ? a->dout_attn : a->dout);
  const int64_t dO_st = gated ? a->dout_attn_stride_t : a->dout_stride_t;
  const int64_t dO_sh = gated ? a->dout_attn_stride_h : a->dout_stride_h;
  {
    KernelTimer tm(a->timer, 4, stream);
    bwd::GateBwd G{static_cast<const bf16*>(a->gate), static_cast<bf16*>(a->dgate), static_cast<bf16*>(a->dout_attn),
                   a->gate_stride_t, a->gate_stride_h, a->dgate_stride_t, a->dgate_stride_h,
                   a->dout_attn_stride_t, a->dout_attn_stride_h};
    const dim3 grid((T + bwd::kPreRows - 1) / bwd::kPreRows);
    if constexpr (HD == 128) {
      if (gated)
        hipLaunchKernelGGL((bwd::prefixlm_bwd_pre_kernel<128, true>), grid, dim3(256), 0, stream,
                           static_cast<const bf16*>(a->out), static_cast<const int8_t*>(a->out_lo),
                           static_cast<const bf16*>(a->dout), a->out_stride_t, a->out_stride_h,
                           a->out_lo_stride_t, a->out_lo_stride_h, a->dout_stride_t, a->dout_stride_h, delta,
                           stats, T, H, a->total_seqlen, G, a->q_amax, q_slots);
    }
    if (!gated)
      hipLaunchKernelGGL((bwd::prefixlm_bwd_pre_kernel<HD, false>), grid, dim3(256), 0, stream,
                         static_cast<const bf16*>(a->out), static_cast<const int8_t*>(a->out_lo),
                         static_cast<const bf16*>(a->dout), a->out_stride_t, a->out_stride_h, a->out_lo_stride_t,
                         a->out_lo_stride_h, a->dout_stride_t, a->dout_stride_h, delta, stats, T, H,
                         a->total_seqlen, G, a->q_amax, q_slots);
  }
  const float scale_log2 = a->softmax_scale * kLog2e;
  if (nkv > 0) {
    bwd::KvParams P;
    P.q = static_cast<const bf16*>(a->q);
    P.k = static_cast<const bf16*>(a->k);
    P.v = static_cast<const bf16*>(a->v);
    P.dout = dO;
    P.lse = a->lse;
    P.delta = delta;
    P.stats = stats;
    P.segstats = segstats;
    P.counters = counters;
    P.ds = nullptr;
    P.ds_scale = nullptr;
    P.ds_base = nullptr;
    P.ds_hbytes = 0;
    P.ds_nkslot = 0;
    if (use_ds) {
      const int64_t hb = ds_cap * 4096;
      P.ds = static_cast<char*>(a->ds_buf);
      P.ds_scale = reinterpret_cast<float*>(P.ds + align_up((size_t)hb * H));
      P.ds_base = ds_base;
      P.ds_hbytes = (uint32_t)hb;
      P.ds_nkslot = (int)ds_nkslot(T, a->numseqs);
    }
    P.dk = static_cast<bf16*>(a->dk);
    P.dv = static_cast<bf16*>(a->dv);
    P.q_st = a->q_stride_t; P.q_sh = a->q_stride_h;
    P.k_st = a->k_stride_t; P.k_sh = a->k_stride_h;
    P.v_st = a->v_stride_t; P.v_sh = a->v_stride_h;
    P.do_st = dO_st; P.do_sh = dO_sh;
    P.dk_st = a->dk_stride_t; P.dk_sh = a->dk_stride_h;
    P.dv_st = a->dv_stride_t; P.dv_sh = a->dv_stride_h;
    P.prefix = a->prefix_lens;
    P.causal = a->causal_lens;
    P.cu = a->cu_seqlens;
    P.items = items_kv;
    P.hdr = hdr_kv;
    P.T = T;
    P.H = H;
    P.is_causal = a->is_causal ? 1 : 0;
    P.numseqs = a->numseqs;
    P.scale_log2 = scale_log2;
    P.scale = a->softmax_scale;
    // persistent: one workgroup per CU (a multiple of 8, see the kernel), fewer when the
    // list is shorter
    int grid = 0;
    rc = persistent_grid(&grid);
    if (rc) return rc;
    const int64_t nblk = std::min<int64_t>(unit_grid(nkv, H), grid);
    KernelTimer tm(a->timer, 5, stream);
    hipLaunchKernelGGL(bwd::prefixlm_bwd_dkdv_kernel<HD>, dim3((unsigned)nblk), dim3(bwd::kv::NT),
                       bwd::kv::Geo<HD>::LDS_BYTES, stream, P);
  }
  if (nq > 0 && use_ds) {
    // dQ = scale dS K from the blocks the dK/dV kernel stored, with its max |K| per
    // (segment, head)
    const int64_t hb = ds_cap * 4096;
    bwd::Q2Params P;
    P.k = static_cast<const bf16*>(a->k);
    P.segstats = segstats;
    P.ds = static_cast<const char*>(a->ds_buf);
    P.ds_scale = reinterpret_cast<const float*>(P.ds + align_up((size_t)hb * H));
    P.ds_base = ds_base;
    P.dq = static_cast<bf16*>(a->dq);
    P.k_st = a->k_stride_t; P.k_sh = a->k_stride_h;
    P.dq_st = a->dq_stride_t; P.dq_sh = a->dq_stride_h;
    P.prefix = a->prefix_lens;
    P.causal = a->causal_lens;
    P.cu = a->cu_seqlens;
    P.items = items_q;
    P.hdr = hdr_q;
    P.T = T;
    P.H = H;
    P.is_causal = a->is_causal ? 1 : 0;
    P.numseqs = a->numseqs;
    P.ds_hbytes = (uint32_t)hb;
    P.ds_nkslot = (int)ds_nkslot(T, a->numseqs);
    P.scale = a->softmax_scale;
    KernelTimer tm(a->timer, 7, stream);
    hipLaunchKernelGGL(bwd::prefixlm_bwd_dq_ds_kernel<HD>, dim3((unsigned)unit_grid(nq, H)), dim3(bwd::q2::NT),
                       bwd::q2::Geo<HD>::LDS_BYTES, stream, P);
  } else if (nq > 0) {
    // reads the per-(segment, head) maxima of |K| and ||V|| the dK/dV kernel wrote
    bwd::QParams P;
    P.q = static_cast<const bf16*>(a->q);
    P.k = static_cast<const bf16*>(a->k);
    P.v = static_cast<const bf16*>(a->v);
    P.dout = dO;
    P.lse = a->lse;
    P.delta = delta;
    P.segstats = segstats;
    P.dq = static_cast<bf16*>(a->dq);
    P.q_st = a->q_stride_t; P.q_sh = a->q_stride_h;
    P.k_st = a->k_stride_t; P.k_sh = a->k_stride_h;
    P.v_st = a->v_stride_t; P.v_sh = a->v_stride_h;
    P.do_st = dO_st; P.do_sh = dO_sh;
    P.dq_st = a->dq_stride_t; P.dq_sh = a->dq_stride_h;
    P.prefix = a->prefix_lens;
    P.causal = a->causal_lens;
    P.cu = a->cu_seqlens;
    P.items = items_q;
    P.hdr = hdr_q;
    P.T = T;
    P.H = H;
    P.is_causal = a->is_causal ? 1 : 0;
    P.numseqs = a->numseqs;
    P.scale_log2 = scale_log2;
    P.scale = a->softmax_scale;
    KernelTimer tm(a->timer, 7, stream);
    hipLaunchKernelGGL(bwd::prefixlm_bwd_dq_kernel<HD>, dim3((unsigned)unit_grid(nq, H)), dim3(bwd::qk::NT),
                       bwd::qk::Geo<HD>::LDS_BYTES, stream, P);
  }
  if (a->total_seqlen < T) {
    KernelTimer tm(a->timer, 6, stream);
    hipLaunchKernelGGL(bwd::prefixlm_bwd_pad_kernel<HD>, dim3((unsigned)(T - a->total_seqlen)), dim3(256), 0,
                       stream, static_cast<bf16*>(a->dq), static_cast<bf16*>(a->dk),
                       static_cast<bf16*>(a->dv), a->dq_stride_t, a->dq_stride_h, a->dk_stride_t,
                       a->dk_stride_h, a->dv_stride_t, a->dv_stride_h, H, a->total_seqlen);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PREFIXLM_ERR_HIP, "backward launch: %s", hipGetErrorString(e));
  return PREFIXLM_OK;
}

extern "C" {

int prefixlm_fwd(const prefixlm_fwd_args* a, void* stream_) {
  if (!a) return fail(PREFIXLM_ERR_INVALID, "args is null");
  // each head dim runs its own instantiation of the forward kernel
  return a->head_dim == 64 ? fwd_launch<64>(a, stream_) : fwd_launch<128>(a, stream_);
}

int prefixlm_bwd(const prefixlm_bwd_args* a, void* stream_) {
  if (!a) return fail(PREFIXLM_ERR_INVALID, "args is null");
  // each head dim runs its own instantiation of the backward kernels
  return a->head_dim == 64 ? bwd_launch<64>(a, stream_) : bwd_launch<128>(a, stream_);
}

size_t prefixlm_bwd_noalloc_max_scratch(void) { return kNoallocScratchBytes; }

int prefixlm_bwd_noalloc(const prefixlm_bwd_args* a, void* stream_) {
  if (!a) return fail(PREFIXLM_ERR_INVALID, "args is null");
  if (a->workspace || a->workspace_bytes)
    return fail(PREFIXLM_ERR_INVALID, "prefixlm_bwd_noalloc uses the library's scratch: workspace must be NULL/0");
  if (a->timer)
    return fail(PREFIXLM_ERR_INVALID, "prefixlm_bwd_noalloc takes no timer (its events would be allocated)");
  const size_t need =
      prefixlm_bwd_workspace_size(a->num_tokens, a->num_heads, a->head_dim, a->total_seqlen, a->numseqs);
  if (need > kNoallocScratchBytes)
    return fail(PREFIXLM_ERR_INVALID,
                "prefixlm_bwd_noalloc: this call needs %zu bytes of scratch, the library's scratch holds %zu "
                "(num_tokens=%d num_heads=%d head_dim=%d numseqs=%d); use prefixlm_bwd with a workspace",
                need, kNoallocScratchBytes, a->num_tokens, a->num_heads, a->head_dim, a->numseqs);
  void* ws = nullptr;
  const int rc = scratch_for_current_device(&ws);
  if (rc) return rc;
  prefixlm_bwd_args b = *a;
  b.workspace = ws;
  b.workspace_bytes = kNoallocScratchBytes;
  return prefixlm_bwd(&b, stream_);
}

int prefixlm_check_workspace(const void* workspace, void* stream_, int32_t* error_word) {
  if (!workspace) return fail(PREFIXLM_ERR_INVALID, "workspace is null");
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  WsHeader h;
  hipError_t e = hipMemcpyAsync(&h, workspace, sizeof(h), hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return fail(PREFIXLM_ERR_HIP, "reading workspace header: %s", hipGetErrorString(e));
  if (error_word) *error_word = h.error;
  if (h.error != 0)
    return fail(PREFIXLM_ERR_METADATA,
                "inconsistent metadata (flags 0x%x): segments must satisfy cu_seqlens[0]=0, "
                "cu_seqlens[s+1]=cu_seqlens[s]+prefix_lens[s]+causal_lens[s] <= total_seqlen",
                h.error);
  return PREFIXLM_OK;
}

int prefixlm_rope(const prefixlm_rope_args* a, void* stream_) {
  if (!a) return fail(PREFIXLM_ERR_INVALID, "args is null");
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (a->head_dim != rope::D) return fail(PREFIXLM_ERR_INVALID, "head_dim must be 128 (got %d)", a->head_dim);
  if (a->num_tokens < 0 || a->num_heads < 1)
    return fail(PREFIXLM_ERR_INVALID, "num_tokens=%d num_heads=%d", a->num_tokens, a->num_heads);
  const void* ptrs[] = {a->x, a->y, a->cos, a->sin};
  for (int i = 0; i < 4; ++i)
    if (!ptrs[i] || !aligned16(ptrs[i]))
      return fail(PREFIXLM_ERR_INVALID, "pointer %d is null or not 16-byte aligned", i);
  const int64_t st[] = {a->x_stride_t, a->x_stride_h, a->y_stride_t, a->y_stride_h};
  for (int i = 0; i < 2; ++i)
    if (st[2 * i] < rope::D || st[2 * i + 1] < 0 || st[2 * i] % 8 || st[2 * i + 1] % 8)
      return fail(PREFIXLM_ERR_INVALID, "tensor %d strides (token %lld, head %lld) must be multiples of 8 "
                  "with token stride >= head_dim", i, (long long)st[2 * i], (long long)st[2 * i + 1]);
  if (a->cs_stride_t < rope::D || a->cs_stride_t % 4)
    return fail(PREFIXLM_ERR_INVALID, "cos/sin row stride %lld must be a multiple of 4 and >= head_dim",
                (long long)a->cs_stride_t);
  const int64_t threads = (int64_t)a->num_tokens * a->num_heads * 8;
  if (threads == 0) return PREFIXLM_OK;
  if ((threads + 255) / 256 > 0x7fffffff) return fail(PREFIXLM_ERR_INVALID, "too many rows");
  rope::Params P{static_cast<const bf16*>(a->x), static_cast<bf16*>(a->y), a->cos, a->sin,
                 a->x_stride_t, a->x_stride_h, a->y_stride_t, a->y_stride_h, a->cs_stride_t,
                 a->num_tokens, a->num_heads, a->backward ? 1 : 0};
  (void)hipGetLastError();
  hipLaunchKernelGGL(rope::rope_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, P);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PREFIXLM_ERR_HIP, "rope launch: %s", hipGetErrorString(e));
  return PREFIXLM_OK;
}

static int swiglu_launch(const prefixlm_swiglu_args* a, void* stream_, bool backward) {
  if (!a) return fail(PREFIXLM_ERR_INVALID, "args is null");
  if (a->rows < 0 || a->cols < 8 || a->cols % 8)
    return fail(PREFIXLM_ERR_INVALID, "rows=%lld cols=%lld: cols must be a positive multiple of 8",
                (long long)a->rows, (long long)a->cols);
  if (a->rows == 0) return PREFIXLM_OK;   // empty tensors may have null pointers
  const void* ptrs[] = {a->gu, backward ? a->dy : a->y, backward ? a->dgu : nullptr};
  for (int i = 0; i < (backward ? 3 : 2); ++i)
    if (!ptrs[i] || !aligned16(ptrs[i]))
      return fail(PREFIXLM_ERR_INVALID, "pointer %d is null or not 16-byte aligned", i);
  const int64_t st[] = {a->gu_stride, backward ? a->dy_stride : a->y_stride, a->dgu_stride};
  const int64_t need[] = {2 * a->cols, a->cols, 2 * a->cols};
  for (int i = 0; i < (backward ? 3 : 2); ++i)
    if (st[i] < need[i] || st[i] % 8)
      return fail(PREFIXLM_ERR_INVALID, "row stride %d (%lld) must be a multiple of 8 and >= %lld", i,
                  (long long)st[i], (long long)need[i]);
  const int64_t threads = a->rows * (a->cols / 8);
  if (threads == 0) return PREFIXLM_OK;
  if ((threads + 255) / 256 > 0x7fffffff) return fail(PREFIXLM_ERR_INVALID, "too many elements");
  nm::SwigluParams P{static_cast<const bf16*>(a->gu), static_cast<const bf16*>(a->dy), static_cast<bf16*>(a->y),
                     static_cast<bf16*>(a->dgu), a->gu_stride, a->y_stride, a->dy_stride, a->dgu_stride,
                     a->rows, a->cols};
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  (void)hipGetLastError();
  hipLaunchKernelGGL(backward ? nm::swiglu_bwd_kernel : nm::swiglu_fwd_kernel, dim3((unsigned)((threads + 255) / 256)),
                     dim3(256), 0, stream, P);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PREFIXLM_ERR_HIP, "swiglu launch: %s", hipGetErrorString(e));
  return PREFIXLM_OK;
}

int prefixlm_swiglu_fwd(const prefixlm_swiglu_args* a, void* stream) { return swiglu_launch(a, stream, false); }
int prefixlm_swiglu_bwd(const prefixlm_swiglu_args* a, void* stream) { return swiglu_launch(a, stream, true); }

// The RMSNorm kernel for rows of `cols` elements: 16-byte chunks per lane, the smallest
// power of two with 64 * nch * 8 >= cols.
static void (*rmsnorm_kernel(int cols, bool backward))(nm::NormParams) {
  const int need = (cols / 8 + 63) / 64;
  int nch = 1;
  while (nch < need) nch *= 2;
  static_assert(nm::kNormMaxChunks == 16, "the dispatch covers up to 16 chunks per lane");
  switch (nch) {
    case 1: return backward ? nm::rmsnorm_bwd_kernel<1> : nm::rmsnorm_fwd_kernel<1>;
    case 2: return backward ? nm::rmsnorm_bwd_kernel<2> : nm::rmsnorm_fwd_kernel<2>;
    case 4: return backward ? nm::rmsnorm_bwd_kernel<4> : nm::rmsnorm_fwd_kernel<4>;
    case 8: return backward ? nm::rmsnorm_bwd_kernel<8> : nm::rmsnorm_fwd_kernel<8>;
    default: return backward ? nm::rmsnorm_bwd_kernel<16> : nm::rmsnorm_fwd_kernel<16>;
  }
}

static int rmsnorm_launch(const prefixlm_rmsnorm_args* a, void* stream_, bool backward) {
  if (!a) return fail(PREFIXLM_ERR_INVALID, "args is null");
  if (a->rows < 0 || a->cols < 8 || a->cols % 8 || a->cols > nm::kNormMaxCols)
    return fail(PREFIXLM_ERR_INVALID, "rows=%lld cols=%d: cols must be a multiple of 8 in [8, %d]",
                (long long)a->rows, a->cols, nm::kNormMaxCols);
  if (!backward && !(a->eps >= 0.f)) return fail(PREFIXLM_ERR_INVALID, "eps must be >= 0");
  if (a->rows == 0) return PREFIXLM_OK;   // empty tensors may have null pointers
  const void* ptrs[] = {a->x, backward ? a->dy : a->y, backward ? a->dx : nullptr};
  for (int i = 0; i < (backward ? 3 : 2); ++i)
    if (!ptrs[i] || !aligned16(ptrs[i]))
      return fail(PREFIXLM_ERR_INVALID, "pointer %d is null or not 16-byte aligned", i);
  if (!a->rstd) return fail(PREFIXLM_ERR_INVALID, "rstd is null");
  const int64_t st[] = {a->x_stride, backward ? a->dy_stride : a->y_stride, a->dx_stride};
  for (int i = 0; i < (backward ? 3 : 2); ++i)
    if (st[i] < a->cols || st[i] % 8)
      return fail(PREFIXLM_ERR_INVALID, "row stride %d (%lld) must be a multiple of 8 and >= cols", i,
                  (long long)st[i]);
  if ((a->rows + 3) / 4 > 0x7fffffff) return fail(PREFIXLM_ERR_INVALID, "too many rows");
  nm::NormParams P{static_cast<const bf16*>(a->x), static_cast<const bf16*>(a->dy), static_cast<bf16*>(a->y),
                   static_cast<bf16*>(a->dx), a->rstd, a->x_stride, a->y_stride, a->dy_stride, a->dx_stride,
                   a->rows, a->cols, a->eps};
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  (void)hipGetLastError();
  hipLaunchKernelGGL(rmsnorm_kernel(a->cols, backward), dim3((unsigned)((a->rows + 3) / 4)), dim3(256), 0, stream, P);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PREFIXLM_ERR_HIP, "rmsnorm launch: %s", hipGetErrorString(e));
  return PREFIXLM_OK;
}

int prefixlm_rmsnorm_fwd(const prefixlm_rmsnorm_args* a, void* stream) { return rmsnorm_launch(a, stream, false); }
int prefixlm_rmsnorm_bwd(const prefixlm_rmsnorm_args* a, void* stream) { return rmsnorm_launch(a, stream, true); }

int prefixlm_proj_gemm(const prefixlm_proj_gemm_args* a, void* stream_) {
  if (!a) return fail(PREFIXLM_ERR_INVALID, "args is null");
  const bool sw = a->swiglu != 0;
  if (a->M < 0 || a->K < mlp::KT || a->K % mlp::KT || a->N < mlp::WT || a->N % mlp::WT)
    return fail(PREFIXLM_ERR_INVALID, "M=%d K=%d N=%d: K must be a positive multiple of %d and N of %d", a->M, a->K,
                a->N, mlp::KT, mlp::WT);
  const int64_t nout = sw ? a->N / 2 : a->N;
  if (a->M == 0) return PREFIXLM_OK;
  const void* ptrs[] = {a->x, a->w, a->y};
  for (int i = 0; i < 3; ++i)
    if (!ptrs[i] || !aligned16(ptrs[i])) return fail(PREFIXLM_ERR_INVALID, "pointer %d is null or not 16-byte aligned", i);
  if (a->x_stride < a->K || a->x_stride % 8 || a->w_stride < a->K || a->w_stride % 8 || a->y_stride < nout ||
      a->y_stride % 8)
    return fail(PREFIXLM_ERR_INVALID, "strides (x %lld, w %lld, y %lld) must be multiples of 8 covering the rows",
                (long long)a->x_stride, (long long)a->w_stride, (long long)a->y_stride);
  if (!(a->eps >= 0.f)) return fail(PREFIXLM_ERR_INVALID, "eps must be >= 0");
  if (a->norm) {
    if (!a->rstd) return fail(PREFIXLM_ERR_INVALID, "norm needs rstd (M floats)");
    if (a->K > nm::kNormMaxCols) return fail(PREFIXLM_ERR_INVALID, "norm: K=%d exceeds %d", a->K, nm::kNormMaxCols);
  }
  // 32-bit byte offsets: within a 256-row tile of x and y, and over all of W
  if ((int64_t)mlp::MT * a->x_stride * 2 >= ((int64_t)1 << 31) ||
      (int64_t)mlp::MT * a->y_stride * 2 >= ((int64_t)1 << 31) || (int64_t)a->N * a->w_stride * 2 >= ((int64_t)1 << 32))
    return fail(PREFIXLM_ERR_INVALID, "operands exceed the 32-bit offsets of the kernel");
  static std::once_flag once;
  static hipError_t attr_err = hipSuccess;
  void (*const kernels[4])(mlp::Params) = {mlp::proj_gemm_kernel<false, false>, mlp::proj_gemm_kernel<false, true>,
                                           mlp::proj_gemm_kernel<true, false>, mlp::proj_gemm_kernel<true, true>};
  std::call_once(once, [&kernels] {
    for (int i = 0; i < 4 && attr_err == hipSuccess; ++i)
      attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(kernels[i]),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, mlp::LDS_BYTES);
  });
  if (attr_err != hipSuccess) return fail(PREFIXLM_ERR_HIP, "hipFuncSetAttribute: %s", hipGetErrorString(attr_err));
  mlp::Params P{static_cast<const bf16*>(a->x), static_cast<const bf16*>(a->w), static_cast<bf16*>(a->y),
                a->rstd, a->x_stride, a->w_stride, a->y_stride, a->M, a->K, a->N, 0, 0};
  P.m_tiles = (a->M + mlp::MT - 1) / mlp::MT;
  P.n_tiles = (int)(sw ? a->N / mlp::WT : a->N / mlp::WT);
  // per XCD: groups of 8 m tiles, each over the n tiles in blocks of 4 (see the kernel)
  const int64_t grid = 8 * (int64_t)((P.m_tiles + 63) / 64) * 8 * ((P.n_tiles + 3) / 4 * 4);
  if (grid > 0x7fffffff) return fail(PREFIXLM_ERR_INVALID, "grid too large");
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  (void)hipGetLastError();
  if (a->norm) {
    // the row scales first (a wave per row, x read once; the normalized x is not written)
    nm::NormParams N{static_cast<const bf16*>(a->x), nullptr, nullptr, nullptr, a->rstd, a->x_stride, 0, 0, 0,
                     a->M, a->K, a->eps};
    hipLaunchKernelGGL(rmsnorm_kernel(a->K, false), dim3((unsigned)((a->M + 3) / 4)), dim3(256), 0, stream, N);
  }
  hipLaunchKernelGGL(kernels[2 * (sw ? 1 : 0) + (a->norm ? 1 : 0)], dim3((unsigned)grid), dim3(mlp::NTH),
                     mlp::LDS_BYTES, stream, P);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PREFIXLM_ERR_HIP, "projection gemm launch: %s", hipGetErrorString(e));
  return PREFIXLM_OK;
}

size_t prefixlm_kvcache_workspace_size(int32_t batch, int32_t seqlen_q, int32_t num_heads, int32_t head_dim,
                                       int32_t max_seqlen_cache) {
  if (batch < 1 || seqlen_q < 1 || num_heads < 1 || max_seqlen_cache < 1) return 0;
  const int64_t nsplit = (max_seqlen_cache + kvc::kChunk - 1) / kvc::kChunk;
  const size_t decode = align_up(sizeof(float) * (size_t)batch * seqlen_q * num_heads * nsplit * kvc::kPart);
  const int64_t T = (int64_t)batch * seqlen_q;
  size_t prefill = 0;
  if (T < 0x7fffffff) {
    prefill = align_up(sizeof(int32_t) * 3 * (size_t)(batch + 1)) +
              align_up(sizeof(float) * (size_t)num_heads * T) +
              prefixlm_fwd_workspace_size((int32_t)T, num_heads, head_dim, (int32_t)T, batch);
  }
  return decode > prefill ? decode : prefill;
}

int prefixlm_kvcache_fwd(const prefixlm_kvcache_args* a, void* stream_) {
  if (!a) return fail(PREFIXLM_ERR_INVALID, "args is null");
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  const int B = a->batch, S = a->seqlen_q, H = a->num_heads, Smax = a->max_seqlen_cache;
  if (a->head_dim != kvc::D) return fail(PREFIXLM_ERR_INVALID, "head_dim must be 128 (got %d)", a->head_dim);
  if (B < 1 || S < 1 || H < 1 || Smax < 1)
    return fail(PREFIXLM_ERR_INVALID, "batch=%d seqlen_q=%d num_heads=%d max_seqlen_cache=%d must be >= 1", B, S,
                H, Smax);
  const bool has_new = a->k != nullptr;
  if ((a->k == nullptr) != (a->v == nullptr)) return fail(PREFIXLM_ERR_INVALID, "k and v must be given together");
  if (!a->cache_seqlens && (a->cache_seqlen < 0 || a->cache_seqlen > Smax))
    return fail(PREFIXLM_ERR_INVALID, "cache_seqlen=%d outside [0, %d]", a->cache_seqlen, Smax);
  const void* ptrs[] = {a->q, a->k_cache, a->v_cache, a->out, a->workspace, a->k, a->v};
  const int nptr = has_new ? 7 : 5;
  for (int i = 0; i < nptr; ++i)
    if (!ptrs[i] || !aligned16(ptrs[i]))
      return fail(PREFIXLM_ERR_INVALID, "tensor pointer %d is null or not 16-byte aligned", i);
  const int64_t st[] = {a->q_stride_b,       a->q_stride_s,       a->q_stride_h,       a->k_cache_stride_b,
                        a->k_cache_stride_s, a->k_cache_stride_h, a->v_cache_stride_b, a->v_cache_stride_s,
                        a->v_cache_stride_h, a->out_stride_b,     a->out_stride_s,     a->out_stride_h,
                        a->k_stride_b,       a->k_stride_s,       a->k_stride_h,       a->v_stride_b,
                        a->v_stride_s,       a->v_stride_h};
  for (int i = 0; i < (has_new ? 18 : 12); ++i)
    if (st[i] < 0 || st[i] % 8)
      return fail(PREFIXLM_ERR_INVALID, "stride %d (%lld) must be a non-negative multiple of 8", i, (long long)st[i]);
  const size_t need = prefixlm_kvcache_workspace_size(B, S, H, a->head_dim, Smax);
  if (a->workspace_bytes < need)
    return fail(PREFIXLM_ERR_INVALID, "workspace of %zu bytes, %zu needed", a->workspace_bytes, need);

  kvc::Params P{};
  P.q = static_cast<const bf16*>(a->q);
  P.k = static_cast<const bf16*>(a->k);
  P.v = static_cast<const bf16*>(a->v);
  P.kc = static_cast<bf16*>(a->k_cache);
  P.vc = static_cast<bf16*>(a->v_cache);
  P.out = static_cast<bf16*>(a->out);
  P.part = static_cast<float*>(a->workspace);
  P.seqlens = a->cache_seqlens;
  P.q_sb = a->q_stride_b; P.q_ss = a->q_stride_s; P.q_sh = a->q_stride_h;
  P.k_sb = a->k_stride_b; P.k_ss = a->k_stride_s; P.k_sh = a->k_stride_h;
  P.v_sb = a->v_stride_b; P.v_ss = a->v_stride_s; P.v_sh = a->v_stride_h;
  P.kc_sb = a->k_cache_stride_b; P.kc_ss = a->k_cache_stride_s; P.kc_sh = a->k_cache_stride_h;
  P.vc_sb = a->v_cache_stride_b; P.vc_ss = a->v_cache_stride_s; P.vc_sh = a->v_cache_stride_h;
  P.o_sb = a->out_stride_b; P.o_ss = a->out_stride_s; P.o_sh = a->out_stride_h;
  P.B = B; P.S = S; P.H = H; P.Smax = Smax;
  P.nsplit = (Smax + kvc::kChunk - 1) / kvc::kChunk;
  P.causal = a->is_causal ? 1 : 0;
  P.seqlen_const = a->cache_seqlen;
  P.s_new = has_new ? S : 0;
  P.scale_log2 = a->softmax_scale * kLog2e;

  (void)hipGetLastError();
  if (has_new) {
    const int64_t threads = (int64_t)B * S * H * 16;
    if ((threads + 255) / 256 > 0x7fffffff) return fail(PREFIXLM_ERR_INVALID, "too many rows");
    hipLaunchKernelGGL(kvc::append_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, P);
  }
  // the reference's prefill: an empty cache and a packed batch of new rows
  const bool packed = B == 1 || (a->q_stride_b == (int64_t)S * a->q_stride_s &&
                                 a->k_stride_b == (int64_t)S * a->k_stride_s &&
                                 a->v_stride_b == (int64_t)S * a->v_stride_s &&
                                 a->out_stride_b == (int64_t)S * a->out_stride_s);
  const int64_t T = (int64_t)B * S;
  if (!a->cache_seqlens && a->cache_seqlen == 0 && has_new && packed && S <= Smax && T < 0x7fffffff &&
      a->q_stride_s >= kvc::D && a->k_stride_s >= kvc::D && a->v_stride_s >= kvc::D && a->out_stride_s >= kvc::D) {
    char* ws = static_cast<char*>(a->workspace);
    int32_t* meta = reinterpret_cast<int32_t*>(ws);
    size_t off = align_up(sizeof(int32_t) * 3 * (size_t)(B + 1));
    float* lse = reinterpret_cast<float*>(ws + off);
    off += align_up(sizeof(float) * (size_t)H * T);
    hipLaunchKernelGGL(kvc::prefill_meta_kernel, dim3(1), dim3(256), 0, stream, meta, meta + (B + 1),
                       meta + 2 * (B + 1), B, S, a->is_causal ? 1 : 0);
    prefixlm_fwd_args f{};
    f.struct_size = sizeof(f);
    f.q = a->q; f.k = a->k; f.v = a->v; f.out = a->out; f.out_lo = nullptr; f.lse = lse;
    f.q_stride_t = a->q_stride_s; f.q_stride_h = a->q_stride_h;
    f.k_stride_t = a->k_stride_s; f.k_stride_h = a->k_stride_h;
    f.v_stride_t = a->v_stride_s; f.v_stride_h = a->v_stride_h;
    f.out_stride_t = a->out_stride_s; f.out_stride_h = a->out_stride_h;
    f.prefix_lens = meta;
    f.causal_lens = meta + (B + 1);
    f.cu_seqlens = meta + 2 * (B + 1);
    f.meta_len = B + 1;
    f.num_tokens = (int32_t)T; f.num_heads = H; f.head_dim = a->head_dim;
    f.total_seqlen = (int32_t)T; f.numseqs = B;
    f.max_seqlen_prefix = a->is_causal ? 0 : S;
    f.max_seqlen_causal = a->is_causal ? S : 0;
    f.max_seqlen_all = S;
    f.is_causal = a->is_causal;
    f.softmax_scale = a->softmax_scale;
    f.workspace = ws + off;
    f.workspace_bytes = a->workspace_bytes - off;
    return prefixlm_fwd(&f, stream_);
  }
  {
    const int64_t nblk = (int64_t)B * H * P.nsplit;
    if (nblk > 0x7fffffff) return fail(PREFIXLM_ERR_INVALID, "grid too large");
    hipLaunchKernelGGL(kvc::decode_kernel, dim3((unsigned)nblk), dim3(kvc::NT), 0, stream, P);
    const int64_t waves = (int64_t)B * S * H;
    hipLaunchKernelGGL(kvc::combine_kernel, dim3((unsigned)((waves * 64 + 255) / 256)), dim3(256), 0, stream, P);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PREFIXLM_ERR_HIP, "kv-cache launch: %s", hipGetErrorString(e));
  return PREFIXLM_OK;
}

size_t prefixlm_plan_size(int32_t total_seqlen, int32_t numseqs) {
  if (total_seqlen < 0 || numseqs < 0) return 0;
  return plan::layout(kPlanLists, total_seqlen, numseqs).bytes;
}

int prefixlm_plan_build(const int32_t* prefix_lens, const int32_t* causal_lens, const int32_t* cu_seqlens,
                        int32_t numseqs, int32_t total_seqlen, int32_t num_tokens, int32_t is_causal,
                        void* plan_out, size_t plan_bytes) {
  if (numseqs < 0 || total_seqlen < 0 || total_seqlen > num_tokens)
    return fail(PREFIXLM_ERR_INVALID, "numseqs=%d, total_seqlen=%d, num_tokens=%d are inconsistent", numseqs,
                total_seqlen, num_tokens);
  if (numseqs > 0 && (!prefix_lens || !causal_lens || !cu_seqlens))
    return fail(PREFIXLM_ERR_INVALID, "metadata pointers must be non-null");
  const plan::Layout l = plan::layout(kPlanLists, total_seqlen, numseqs);
  if (!plan_out || plan_bytes != l.bytes)
    return fail(PREFIXLM_ERR_INVALID, "plan buffer of %zu bytes, %zu needed", plan_bytes, l.bytes);
  const int32_t err = plan::build(kPlanLists, l, prefix_lens, causal_lens, cu_seqlens, numseqs, total_seqlen,
                                  num_tokens, is_causal ? 1 : 0, static_cast<unsigned char*>(plan_out));
  if (err)
    return fail(PREFIXLM_ERR_METADATA,
                "inconsistent metadata (flags 0x%x): segments must satisfy cu_seqlens[0]=0, "
                "cu_seqlens[s+1]=cu_seqlens[s]+prefix_lens[s]+causal_lens[s] <= total_seqlen",
                err);
  return PREFIXLM_OK;
}

int64_t prefixlm_plan_ds_blocks(const void* plan_p, size_t plan_bytes) {
  if (!plan_p || plan_bytes < sizeof(WsHeader)) return -1;
  WsHeader h;
  memcpy(&h, plan_p, sizeof(h));
  if (h.pad[0] != plan::kPlanMagic || h.pad[1] < 0 || h.pad[2] < 0) return -1;
  if (plan::layout(kPlanLists, h.pad[2], h.pad[1]).bytes != plan_bytes) return -1;
  return h.pad[4];
}

void* prefixlm_timer_create(void) { return new (std::nothrow) prefixlm_timer(); }

void prefixlm_timer_destroy(void* timer) {
  prefixlm_timer* t = static_cast<prefixlm_timer*>(timer);
  if (!t) return;
  for (auto& r : t->recs) {
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  for (hipEvent_t e : t->pool) (void)hipEventDestroy(e);
  delete t;
}

int prefixlm_timer_read(void* timer, float* total_ms, int32_t* launches) {
  prefixlm_timer* t = static_cast<prefixlm_timer*>(timer);
  if (!t) return fail(PREFIXLM_ERR_INVALID, "timer is null");
  for (int i = 0; i < PREFIXLM_NUM_KERNELS; ++i) {
    if (total_ms) total_ms[i] = 0.f;
    if (launches) launches[i] = 0;
  }
  int rc = PREFIXLM_OK;
  for (auto& r : t->recs) {
    float ms = 0.f;
    hipError_t e = hipEventSynchronize(r.b);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.a, r.b);
    if (e != hipSuccess) {
      rc = fail(PREFIXLM_ERR_HIP, "timing event: %s", hipGetErrorString(e));
    } else if (r.id >= 0 && r.id < PREFIXLM_NUM_KERNELS) {
      if (total_ms) total_ms[r.id] += ms;
      if (launches) launches[r.id] += 1;
    }
    t->pool.push_back(r.a);
    t->pool.push_back(r.b);
  }
  t->recs.clear();
  return rc;
}

}  // extern "C"
