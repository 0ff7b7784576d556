// jn_propagation_topk_forward_static: the top-k propagation forward with its
// scratch in a file-scope device array instead of a caller workspace, for
// callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc).  The kernels are
// jn_propagation_topk_forward's; only where the select's split key rows live
// differs.
//
// `scratch` is one fixed array per device (each GPU the library runs on holds
// it until the process ends).  Host code never passes the array's name to a
// kernel: on the host it is a stand-in symbol, not a device address.  The
// device address comes from hipGetSymbolAddress, once per device with that
// device current, and is kept per device.  Every call on a GPU shares that
// GPU's array and leaves the last call's contents in it; calls that overlap on
// one GPU (other streams, other host threads) race on it.  Nothing in it has
// to start at zero: the select's prep kernels write every byte they later read.
#include <mutex>

#include "../../include/jakal_net_hip.h"
#include "jn_internal.hpp"

namespace {

// Holds the split-fp16 key rows of B*N keys of rank r (B*N*RP*4 bytes, RP = r
// rounded up to 32) plus per-batch scale exponents and per-block maxima: 48 MiB
// covers the C4 workload (B=16, N=4096, r=64: 16.8 MB) up to B*N = 196,608
// keys at rank <= 64, or 98,304 at rank <= 128.
constexpr size_t kStaticScratchBytes = size_t(48) << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device (looked up once per device).
int device_scratch(void** out) {
  int dev = -1;
  JN_HIP_TRY(hipGetDevice(&dev));
  JN_REQUIRE(dev >= 0 && dev < kMaxDevices, jakal::kUnsupported, "device ordinal %d beyond the %d supported", dev,
             kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    JN_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    JN_REQUIRE(p != nullptr, jakal::kHipError, "hipGetSymbolAddress returned no address for the static scratch");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return jakal::kOk;
}

}  // namespace

extern "C" {

size_t jn_static_scratch_bytes(void) { return kStaticScratchBytes; }

int jn_propagation_topk_forward_static(const float* layer_val, const float* projected_state,
                                       const float* projected_val, const float* target_weight,
                                       const float* source_weight, const float* core_weight, const float* bias,
                                       int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
                                       int64_t topk, int32_t compress_kind, float* delta_state, float* delta_val,
                                       float* projections, int32_t* topk_index, float* topk_score,
                                       jn_stream_t stream) {
  // sizes are checked before the device is touched
  JN_REQUIRE(batch >= 1 && nodes >= 1 && rank >= 1, jakal::kInvalidArgument,
             "batch, nodes and rank must be positive (B=%lld N=%lld r=%lld)", (long long)batch, (long long)nodes,
             (long long)rank);
  const size_t need = jn_propagation_topk_forward_workspace_bytes(batch, nodes, rank);
  JN_REQUIRE(need <= kStaticScratchBytes, jakal::kUnsupported,
             "jn_propagation_topk_forward_static: B=%lld, N=%lld, rank %lld need %zu bytes of scratch; the static "
             "scratch holds %zu (use jn_propagation_topk_forward with a workspace)",
             (long long)batch, (long long)nodes, (long long)rank, need, kStaticScratchBytes);
  void* ws = nullptr;
  const int rc = device_scratch(&ws);
  if (rc) return rc;
  return jn_propagation_topk_forward(layer_val, projected_state, projected_val, target_weight, source_weight,
                                     core_weight, bias, batch, nodes, in_dim, out_dim, rank, topk, compress_kind,
                                     delta_state, delta_val, projections, topk_index, topk_score, nullptr, 0, ws,
                                     kStaticScratchBytes, stream);
}

}  // extern "C"
