// mx_qdense_noalloc: FusedQuantizedDense on device pointers without any device allocation, for
// callers that cannot allocate (HIP graph capture, serving loops, harnesses that forbid
// hipMalloc).  It runs mx_qdense's own kernels; only where they keep state between workgroups
// does the memory differ:
//
//   - the split-K partial tiles and arrival counters of the skinny and GEMV kernels come from
//     `scratch`, a static device array of MX_QDENSE_NOALLOC_SCRATCH_BYTES that every GPU the
//     library runs on holds until the process ends, instead of the backend's growable scratch;
//     a problem that needs more is rejected before anything is launched;
//   - a problem that mx_qdense would compute through a dequantised f32 copy of the weights runs
//     the exact kernel, which needs no workspace;
//   - any other device allocation reached during the call is an error (dev_alloc refuses it).
//
// Layout of `scratch` (the same as the backend's scratch): bytes [0, 64 KiB) are the arrival
// counters, one per column block, which must be zero between launches (the last workgroup of a
// column block resets its own); the partial tiles [S, M, N] f32 follow.  The counters are cleared
// once per device, here, at set-up; the partial tiles are written before they are read.
//
// Every call on one GPU shares that GPU's array, from any backend, and the array keeps the last
// call's contents: calls that overlap on one GPU (several streams or backends) race.
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
    return MX_OK;
  }
  void* ptr = nullptr;
  hipError_t e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || ptr == nullptr)
    return set_error(MX_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d failed: %s", b->device,
                     hipGetErrorString(e));
  // The counters start at zero.  The stream is synchronised so that work on any other stream of
  // this device sees the cleared counters.
  const int words = (int)(kCounterBytes / 4);
  hipLaunchKernelGGL(clear_words, dim3((words + 255) / 256), dim3(256), 0, b->stream, (uint32_t*)ptr, words);
  MX_CHECK_HIP(hipGetLastError());
  MX_CHECK_HIP(hipStreamSynchronize(b->stream));
  g_scratch_ptr[b->device] = ptr;
  b->noalloc_scratch = ptr;
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
  struct Scope {
    mx_backend* b;
    explicit Scope(mx_backend* bb) : b(bb) { b->noalloc_active = true; }
    ~Scope() { b->noalloc_active = false; }
  } scope(b);
  return mx::qdense_run(b, d);
}
