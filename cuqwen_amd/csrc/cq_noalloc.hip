// Allocation-free decode attention: cq_gqa_attention_decode with its split-K
// partials in a file-scope device array instead of a caller workspace, for
// callers that cannot allocate (code under HIP graph capture, serving loops
// that forbid hipMalloc).  No counterpart in the reference.
//
// `scratch` is a host-side stand-in in host code: its device address comes
// from hipGetSymbolAddress, once per device, with that device current, and
// only that address is handed to kernels.  Every call on a device shares the
// device's copy; nothing in it has to start at zero (the merge reads only the
// partitions the current call's stage 1 wrote), and calls that overlap on one
// device race.
#include <mutex>

#include "cq_internal.h"

namespace cq {

// Partials of the largest shape the attention accepts: n_kv_heads <= 64
// gives at most 256 + 63 (kv head, partition) blocks of 16 head slots, each
// (max, sum, 128 output dims) fp32 -- 2,653,440 bytes; rounded up.
constexpr size_t kNoAllocScratchBytes = 2816u * 1024u;
constexpr int kNoAllocMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kNoAllocMaxDevices];

static int scratch_ptr(void** out) {
  int dev = -1;
  CQ_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kNoAllocMaxDevices) return fail(CQ_EINVAL, "noalloc attention: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(CQ_EHIP, std::string("noalloc attention: hipGetSymbolAddress: ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return CQ_OK;
}

}  // namespace cq

using namespace cq;

extern "C" size_t cq_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int cq_gqa_attention_decode_noalloc(const void* q, const void* kc, const void* vc, void* out,
                                               const int32_t* d_pos, int32_t n_heads, int32_t n_kv_heads,
                                               int32_t head_dim, int32_t max_seq_len, void* stream) {
  if (n_kv_heads <= 0 || head_dim <= 0) return fail(CQ_EINVAL, "noalloc attention: bad shape");
  const size_t need = attention_workspace_bytes(n_heads, n_kv_heads, head_dim);
  if (need > kNoAllocScratchBytes)
    return fail(CQ_ERANGE, "noalloc attention: partials of " + std::to_string(need) + " bytes exceed the " +
                               std::to_string(kNoAllocScratchBytes) + "-byte scratch");
  void* ws = nullptr;
  CQ_TRY(scratch_ptr(&ws));
  AttnArgs a;
  a.q = (const __half*)q; a.kcache = (const __half*)kc; a.vcache = (const __half*)vc; a.out = (__half*)out;
  a.d_pos = d_pos; a.n_heads = n_heads; a.n_kv = n_kv_heads; a.head_dim = head_dim; a.max_seq = max_seq_len;
  a.workspace = ws;
  return launch_attention(a, static_cast<hipStream_t>(stream));
}
