// mx_qdense_noalloc: FusedQuantizedDense on device pointers without any device allocation, for
// callers that cannot allocate (HIP graph capture, serving loops, harnesses that forbid
// hipMalloc).  It runs mx_qdense's own kernels; only where they keep state between workgroups
// does the memory differ:
//
//   - the split-K partial tiles and arrival counters of the skinny and GEMV kernels come from
//     `scratch`, a static device array of MX_QDENSE_NOALLOC_SCRATCH_BYTES that every GPU the
//     library runs on holds until the process ends, instead of the backend's growable scratch;
//     a problem that needs more is rejected before anything is launched;
//   - GGML rows past 20 rows, which mx_qdense dequantises into an f32 copy for the f32 matrix
//     cores, run the decode GEMV once per group of four rows instead;
//   - any other device allocation reached during the call is an error (dev_alloc refuses it).
//
// Layout of `scratch` (the same as the backend's scratch): bytes [0, 64 KiB) are the arrival
// counters, one per column block, which must be zero between launches (the last workgroup of a
// column block resets its own); the partial tiles [S, M, N] f32 follow.  The counters are cleared
// once per device, here, at set-up; the partial tiles are written before they are read.
//
// Every call on one GPU shares that GPU's array, from any backend, and the array keeps the last
// call's contents.  Calls are therefore ordered on the device: each call's stream first waits
// for the previous call's completion event (recorded on whichever stream that call used), then
// launches, then records the event again, all under a per-device lock.  Calls from several
// streams or backends thus run one after another without allocating.  A stream under graph
// capture is the exception: capture cannot wait on an event recorded outside the graph, so a
// captured call is ordered only by the caller; a captured graph replayed while another noalloc
// call runs on the same GPU races with it, and the counters it disturbs can then make later calls
// on that GPU wrong as well.
#include <map>
#include <mutex>

#include "mxrt_internal.h"

namespace mx {

static __device__ __align__(256) unsigned char scratch[MX_QDENSE_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr size_t kCounterBytes = 64 * 1024;  // the skinny and GEMV kernels' counter region
static_assert(MX_QDENSE_NOALLOC_SCRATCH_BYTES > kCounterBytes, "scratch holds the counters");

std::mutex g_mu;
std::map<int, void*> g_scratch_ptr;  // device -> that device's address of `scratch`

// Per-device ordering of the calls that share `scratch`.
struct Order {
  std::mutex mu;
  hipEvent_t done = nullptr;  // completion of the last call (valid once `used`)
  bool used = false;
};
std::map<int, Order*> g_order;  // device -> ordering state (created at set-up, never freed)

__global__ void clear_words(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

}  // namespace

int noalloc_scratch_setup(mx_backend* b) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_scratch_ptr.find(b->device);
  if (it != g_scratch_ptr.end()) {
    b->noalloc_scratch = it->second;
    b->noalloc_order = g_order[b->device];
    return MX_OK;
  }
  Order* ord = new Order;
  if (hipError_t ee = hipEventCreateWithFlags(&ord->done, hipEventDisableTiming); ee != hipSuccess) {
    delete ord;
    return set_error(MX_ERR_HIP, "hipEventCreate for mx_qdense_noalloc on device %d failed: %s", b->device,
                     hipGetErrorString(ee));
  }
  // On failure the ordering state is released again (nothing has been published yet).
  auto fail = [&](const char* what, hipError_t err) {
    hipEventDestroy(ord->done);
    delete ord;
    return set_error(MX_ERR_HIP, "%s for mx_qdense_noalloc on device %d failed: %s", what, b->device,
                     hipGetErrorString(err));
  };
  void* ptr = nullptr;
  hipError_t e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || ptr == nullptr) return fail("hipGetSymbolAddress(scratch)", e);
  // The counters start at zero.  The stream is synchronised so that work on any other stream of
  // this device sees the cleared counters.
  const int words = (int)(kCounterBytes / 4);
  hipLaunchKernelGGL(clear_words, dim3((words + 255) / 256), dim3(256), 0, b->stream, (uint32_t*)ptr, words);
  if ((e = hipGetLastError()) != hipSuccess) return fail("clearing the counters", e);
  if ((e = hipStreamSynchronize(b->stream)) != hipSuccess) return fail("clearing the counters", e);
  g_scratch_ptr[b->device] = ptr;
  g_order[b->device] = ord;
  b->noalloc_scratch = ptr;
  b->noalloc_order = ord;
  return MX_OK;
}

}  // namespace mx

extern "C" int mx_qdense_noalloc(mx_backend* b, const mx_qdense_args* args) {
  mx::clear_error();
  MX_TRY(mx::check_device(b));
  if (!b->noalloc_scratch)
    return mx::set_error(MX_ERR_INVALID, "mx_qdense_noalloc: no static scratch on device %d", b->device);
  mx::QDenseDesc d;
  MX_TRY(mx::qdense_validate(args, &d));
  std::lock_guard<std::recursive_mutex> lk(b->mu);
  auto* ord = static_cast<mx::Order*>(b->noalloc_order);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  MX_CHECK_HIP(hipStreamIsCapturing(b->stream, &cs));
  const bool ordered = cs == hipStreamCaptureStatusNone;
  std::unique_lock<std::mutex> olk(ord->mu, std::defer_lock);
  if (ordered) {
    olk.lock();
    // Wait for the previous call on this GPU, from any stream or backend (a no-op when it was
    // on this stream, whose order already holds).
    if (ord->used) MX_CHECK_HIP(hipStreamWaitEvent(b->stream, ord->done, 0));
  }
  int rc;
  {
    struct Scope {
      mx_backend* b;
      explicit Scope(mx_backend* bb) : b(bb) { b->noalloc_active = true; }
      ~Scope() { b->noalloc_active = false; }
    } scope(b);
    rc = mx::qdense_run(b, d);
  }
  if (ordered) {
    // Recorded even after a failed launch, so that the next call still waits for whatever this
    // one queued.
    MX_CHECK_HIP(hipEventRecord(ord->done, b->stream));
    ord->used = true;
  }
  return rc;
}

extern "C" int mx_backend_debug_noalloc_scratch(const mx_backend* b, void** out) {
  mx::clear_error();
  if (!b || !out) return mx::set_error(MX_ERR_INVALID, "mx_backend_debug_noalloc_scratch: null argument");
  *out = b->noalloc_scratch;
  return MX_OK;
}
