// Runtime of the MI355X backend: device context, caching allocator, buffers, errors, timing.
//
// Mirrors the reference's compute.Backend / compute.Buffer contracts (compute.go:68-102,
// buffer.go:12-61) with device-resident storage: a buffer lives in HBM from
// BufferFromFlatData until Finalize, and Execute never copies inputs back to the host.

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <string>

#include "mxrt_internal.h"

namespace mx {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

// ---------------------------------------------------------------------------------------------
// DTypes.
// ---------------------------------------------------------------------------------------------
bool dtype_known(int dt) { return dtype_bits(dt) > 0; }

const char* dtype_name(int dt) {
  switch (dt) {
    case MX_DTYPE_BOOL: return "Bool";
    case MX_DTYPE_INT8: return "Int8";
    case MX_DTYPE_INT16: return "Int16";
    case MX_DTYPE_INT32: return "Int32";
    case MX_DTYPE_INT64: return "Int64";
    case MX_DTYPE_UINT8: return "Uint8";
    case MX_DTYPE_UINT16: return "Uint16";
    case MX_DTYPE_UINT32: return "Uint32";
    case MX_DTYPE_UINT64: return "Uint64";
    case MX_DTYPE_FLOAT16: return "Float16";
    case MX_DTYPE_FLOAT32: return "Float32";
    case MX_DTYPE_FLOAT64: return "Float64";
    case MX_DTYPE_BFLOAT16: return "BFloat16";
    case MX_DTYPE_INT4: return "Int4";
    case MX_DTYPE_UINT4: return "Uint4";
    default: return "InvalidDType";
  }
}

int dtype_bits(int dt) {
  switch (dt) {
    case MX_DTYPE_BOOL:
    case MX_DTYPE_INT8:
    case MX_DTYPE_UINT8: return 8;
    case MX_DTYPE_INT16:
    case MX_DTYPE_UINT16:
    case MX_DTYPE_FLOAT16:
    case MX_DTYPE_BFLOAT16: return 16;
    case MX_DTYPE_INT32:
    case MX_DTYPE_UINT32:
    case MX_DTYPE_FLOAT32: return 32;
    case MX_DTYPE_INT64:
    case MX_DTYPE_UINT64:
    case MX_DTYPE_FLOAT64: return 64;
    case MX_DTYPE_INT4:
    case MX_DTYPE_UINT4: return 4;
    default: return 0;
  }
}

bool dtype_is_float(int dt) {
  return dt == MX_DTYPE_FLOAT16 || dt == MX_DTYPE_BFLOAT16 || dt == MX_DTYPE_FLOAT32 ||
         dt == MX_DTYPE_FLOAT64;
}
bool dtype_is_half(int dt) { return dt == MX_DTYPE_FLOAT16 || dt == MX_DTYPE_BFLOAT16; }
bool dtype_is_int(int dt) {
  switch (dt) {
    case MX_DTYPE_INT8: case MX_DTYPE_INT16: case MX_DTYPE_INT32: case MX_DTYPE_INT64:
    case MX_DTYPE_UINT8: case MX_DTYPE_UINT16: case MX_DTYPE_UINT32: case MX_DTYPE_UINT64:
    case MX_DTYPE_INT4: case MX_DTYPE_UINT4:
      return true;
    default:
      return false;
  }
}
bool dtype_is_packed(int dt) { return dt == MX_DTYPE_INT4 || dt == MX_DTYPE_UINT4; }

std::string Shape::str() const {
  std::string s = "(";
  s += dtype_name(dtype);
  if (!dims.empty()) {
    s += ")[";
    for (size_t i = 0; i < dims.size(); ++i) {
      if (i) s += " ";
      s += std::to_string(dims[i]);
    }
    s += "]";
  } else {
    s += ")";
  }
  return s;
}

int shape_from_c(const mx_shape* s, Shape* out) {
  if (!s) return set_error(MX_ERR_INVALID, "shape is NULL");
  if (!dtype_known(s->dtype)) return set_error(MX_ERR_INVALID, "unsupported dtype %d", s->dtype);
  if (s->rank < 0 || s->rank > MX_MAX_RANK)
    return set_error(MX_ERR_INVALID, "rank %d out of range [0, %d]", s->rank, MX_MAX_RANK);
  out->dtype = s->dtype;
  out->dims.assign(s->dims, s->dims + s->rank);
  for (auto d : out->dims)
    if (d < 0) return set_error(MX_ERR_INVALID, "negative dimension in shape %s", out->str().c_str());
  return MX_OK;
}

void shape_to_c(const Shape& s, mx_shape* out) {
  memset(out, 0, sizeof(*out));
  out->dtype = s.dtype;
  out->rank = s.rank();
  for (int i = 0; i < s.rank() && i < MX_MAX_RANK; ++i) out->dims[i] = s.dims[i];
}

// ---------------------------------------------------------------------------------------------
// Caching device allocator.
// ---------------------------------------------------------------------------------------------
size_t DevicePool::round_size(size_t b) {
  if (b == 0) b = 1;
  if (b <= (1u << 20)) return (b + 255) & ~size_t(255);
  return (b + (1u << 16) - 1) & ~size_t((1u << 16) - 1);  // 64 KiB granularity above 1 MiB
}

int DevicePool::alloc(size_t bytes, void** out) {
  if (fail_after > 0) {
    if (--fail_after == 0)
      return set_error(MX_ERR_OUT_OF_MEMORY, "device allocation of %zu bytes failed (injected)", bytes);
  }
  size_t r = round_size(bytes);
  auto it = free_.find(r);
  if (it != free_.end()) {
    *out = it->second;
    free_.erase(it);
    cached_ -= r;
    live_[*out] = r;
    in_use_ += r;
    return MX_OK;
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, r);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    trim();
    e = hipMalloc(&p, r);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return set_error(MX_ERR_OUT_OF_MEMORY, "hipMalloc(%zu) failed: %s", r, hipGetErrorString(e));
    }
  }
  live_[p] = r;
  in_use_ += r;
  *out = p;
  return MX_OK;
}

void DevicePool::release(void* p) {
  if (!p) return;
  auto it = live_.find(p);
  if (it == live_.end()) return;
  size_t r = it->second;
  live_.erase(it);
  in_use_ -= r;
  free_.emplace(r, p);
  cached_ += r;
}

void DevicePool::trim() {
  for (auto& kv : free_) (void)hipFree(kv.second);
  free_.clear();
  cached_ = 0;
}

void DevicePool::destroy() {
  trim();
  for (auto& kv : live_) (void)hipFree(kv.first);
  live_.clear();
  in_use_ = 0;
}

int check_device(mx_backend* b) {
  if (!b) return set_error(MX_ERR_INVALID, "backend is NULL");
  if (b->finalized) return set_error(MX_ERR_FINALIZED, "backend already finalized");
  if (b->host_only) return set_error(MX_ERR_NO_DEVICE, "backend opened host_only: no device operations");
  return MX_OK;
}

int dev_alloc(mx_backend* b, size_t bytes, void** out) {
  MX_TRY(check_device(b));
  if (b->noalloc_active)
    return set_error(MX_ERR_INVALID, "mx_qdense_noalloc: this problem would allocate %zu bytes of device memory",
                     bytes);
  return b->pool.alloc(bytes, out);
}

void dev_free(mx_backend* b, void* p) {
  if (b && !b->finalized && !b->host_only) b->pool.release(p);
}

int ensure_scratch(mx_backend* b, size_t bytes, void** out) {
  if (b->noalloc_active) {
    if (bytes > MX_QDENSE_NOALLOC_SCRATCH_BYTES)
      return set_error(MX_ERR_INVALID,
                       "mx_qdense_noalloc: the split-K scratch of this problem (%zu bytes) exceeds the "
                       "static maximum of %u bytes; use mx_qdense",
                       bytes, (unsigned)MX_QDENSE_NOALLOC_SCRATCH_BYTES);
    *out = b->noalloc_scratch;
    return MX_OK;
  }
  if (b->scratch_bytes < bytes) {
    if (b->scratch) {
      MX_CHECK_HIP(hipStreamSynchronize(b->stream));
      (void)hipFree(b->scratch);
      b->scratch = nullptr;
      b->scratch_bytes = 0;
    }
    size_t want = std::max(bytes, (size_t)(8u << 20));
    MX_CHECK_HIP(hipMalloc(&b->scratch, want));
    MX_CHECK_HIP(hipMemsetAsync(b->scratch, 0, want, b->stream));
    b->scratch_bytes = want;
  }
  *out = b->scratch;
  return MX_OK;
}

// ---------------------------------------------------------------------------------------------
// Host waits.  A blocking wait lets the calling thread sleep until the runtime wakes it, which
// after a wait of a few tens of microseconds costs about as much again; the waits below poll the
// stream or event for up to kSpinWaitMs, keeping the thread on its core so it returns (and issues
// its next launches) as soon as the work is done, then fall back to the blocking wait so that a
// long wait does not occupy a core.
// ---------------------------------------------------------------------------------------------
constexpr double kSpinWaitMs = 2.0;

static double now_ms() {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

hipError_t wait_stream(hipStream_t st) {
  const double t0 = now_ms();
  for (;;) {
    const hipError_t e = hipStreamQuery(st);
    if (e != hipErrorNotReady) return e;
    if (now_ms() - t0 > kSpinWaitMs) return hipStreamSynchronize(st);
  }
}

static hipError_t wait_event(hipEvent_t ev) {
  const double t0 = now_ms();
  for (;;) {
    const hipError_t e = hipEventQuery(ev);
    if (e != hipErrorNotReady) return e;
    if (now_ms() - t0 > kSpinWaitMs) return hipEventSynchronize(ev);
  }
}

// ---------------------------------------------------------------------------------------------
// Timing.
// ---------------------------------------------------------------------------------------------
static int get_event(mx_backend* b, hipEvent_t* ev) {
  if (!b->event_cache.empty()) {
    *ev = b->event_cache.back();
    b->event_cache.pop_back();
    return MX_OK;
  }
  MX_CHECK_HIP(hipEventCreate(ev));
  return MX_OK;
}

thread_local LaunchEvents g_launch_events;

int timing_begin(mx_backend* b, LaunchEvents* ev) {
  MX_TRY(get_event(b, &ev->start));
  MX_TRY(get_event(b, &ev->stop));
  return MX_OK;
}

int timing_end(mx_backend* b, const char* name, const LaunchEvents& ev) {
  b->pending.push_back(PendingTiming{name, ev.start, ev.stop});
  return MX_OK;
}

static int resolve_timings(mx_backend* b) {
  if (b->pending.empty()) return MX_OK;
  MX_CHECK_HIP(hipStreamSynchronize(b->stream));
  for (auto& p : b->pending) {
    float ms = 0.f;
    MX_CHECK_HIP(hipEventElapsedTime(&ms, p.start, p.stop));
    auto& e = b->prof[p.name];
    e.launches += 1;
    e.total_ms += ms;
    b->event_cache.push_back(p.start);
    b->event_cache.push_back(p.stop);
  }
  b->pending.clear();
  return MX_OK;
}

}  // namespace mx

using namespace mx;

// ===============================================================================================
// C ABI.
// ===============================================================================================
extern "C" {

const char* mx_last_error(void) { return g_last_error.c_str(); }

static void copy_str(const std::string& s, char* buf, size_t len) {
  if (!buf || len == 0) return;
  size_t n = std::min(len - 1, s.size());
  memcpy(buf, s.data(), n);
  buf[n] = 0;
}

int mx_backend_new(const char* config, mx_backend** out) {
  clear_error();
  if (!out) return set_error(MX_ERR_INVALID, "out is NULL");
  *out = nullptr;
  std::string cfg = config ? config : "";
  int device = 0;
  bool host_only = false, no_fusion = false, exact = false, gemv_over_gemm = false;
  // Comma-separated options, mirroring the "name:cfg" convention of GOMLX_BACKEND (compute.go:141-147).
  size_t pos = 0;
  while (pos <= cfg.size()) {
    size_t comma = cfg.find(',', pos);
    std::string opt = cfg.substr(pos, comma == std::string::npos ? std::string::npos : comma - pos);
    if (opt == "host_only") {
      host_only = true;
    } else if (opt == "nofusion") {
      no_fusion = true;
    } else if (opt == "exact") {
      exact = true;
    } else if (opt == "gemv_over_gemm") {
      gemv_over_gemm = true;
    } else if (opt.rfind("device=", 0) == 0) {
      char* end = nullptr;
      long v = strtol(opt.c_str() + 7, &end, 10);
      if (!end || *end || v < 0) return set_error(MX_ERR_INVALID, "bad device option \"%s\"", opt.c_str());
      device = (int)v;
    } else if (!opt.empty()) {
      return set_error(MX_ERR_INVALID, "unknown mi355x backend option \"%s\"", opt.c_str());
    }
    if (comma == std::string::npos) break;
    pos = comma + 1;
  }
  auto* b = new mx_backend();
  b->device = device;
  b->host_only = host_only;
  b->no_fusion = no_fusion;
  b->exact_qdense = exact;
  b->gemv_over_gemm = gemv_over_gemm;
  if (host_only) {
    b->description = "MI355X backend (host_only: graph building only)";
    *out = b;
    return MX_OK;
  }
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0) {
    (void)hipGetLastError();
    delete b;
    return set_error(MX_ERR_NO_DEVICE, "no HIP device available (%s)",
                     e == hipSuccess ? "0 devices" : hipGetErrorString(e));
  }
  if (device >= count) {
    delete b;
    return set_error(MX_ERR_INVALID, "device %d out of range (%d devices)", device, count);
  }
  e = hipSetDevice(device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking);
  hipDeviceProp_t prop;
  if (e == hipSuccess) e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) {
    if (b->stream) (void)hipStreamDestroy(b->stream);
    delete b;
    return set_error(MX_ERR_HIP, "device init failed: %s", hipGetErrorString(e));
  }
  if (int rc = noalloc_scratch_setup(b); rc != MX_OK) {
    (void)hipStreamDestroy(b->stream);
    delete b;
    return rc;
  }
  b->num_cus = prop.multiProcessorCount;
  char desc[512];
  snprintf(desc, sizeof(desc), "%s (%s), %d CUs, %.1f GiB HBM", prop.name, prop.gcnArchName,
           prop.multiProcessorCount, prop.totalGlobalMem / double(1u << 30));
  b->description = desc;
  *out = b;
  return MX_OK;
}

int mx_backend_finalize(mx_backend* b) {
  clear_error();
  if (!b) return MX_OK;
  std::lock_guard<std::recursive_mutex> lk(b->mu);
  if (b->finalized) return MX_OK;
  if (!b->host_only) {
    (void)hipSetDevice(b->device);
    if (b->stream) (void)hipStreamSynchronize(b->stream);
    for (auto& p : b->pending) {
      (void)hipEventDestroy(p.start);
      (void)hipEventDestroy(p.stop);
    }
    b->pending.clear();
    for (auto ev : b->event_cache) (void)hipEventDestroy(ev);
    b->event_cache.clear();
    if (b->region_start) (void)hipEventDestroy(b->region_start);
    if (b->region_stop) (void)hipEventDestroy(b->region_stop);
    b->region_start = b->region_stop = nullptr;
    if (b->scratch) (void)hipFree(b->scratch);
    b->scratch = nullptr;
    b->pool.destroy();
    if (b->stream) (void)hipStreamDestroy(b->stream);
    b->stream = nullptr;
  }
  b->finalized = true;
  // The handle itself stays allocated so IsFinalized and the buffers that still point at it
  // keep working (compute.go:97-101).
  return MX_OK;
}

int mx_backend_is_finalized(const mx_backend* b) { return b ? (b->finalized ? 1 : 0) : 1; }

int mx_backend_name(const mx_backend* b, char* buf, size_t buflen) {
  clear_error();
  if (!b) return set_error(MX_ERR_INVALID, "backend is NULL");
  copy_str("mi355x", buf, buflen);
  return MX_OK;
}

int mx_backend_description(const mx_backend* b, char* buf, size_t buflen) {
  clear_error();
  if (!b) return set_error(MX_ERR_INVALID, "backend is NULL");
  copy_str("mi355x: MI355X-native compute backend — " + b->description, buf, buflen);
  return MX_OK;
}

int mx_backend_num_devices(const mx_backend* b, int* out) {
  clear_error();
  if (!b || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  *out = b->host_only ? 0 : 1;  // one process drives one GPU
  return MX_OK;
}

int mx_backend_device_description(const mx_backend* b, int device, char* buf, size_t buflen) {
  clear_error();
  if (!b) return set_error(MX_ERR_INVALID, "backend is NULL");
  if (b->host_only || device != 0) return set_error(MX_ERR_INVALID, "device %d not available", device);
  copy_str(b->description, buf, buflen);
  return MX_OK;
}

int mx_backend_supports_dtype(const mx_backend* b, int dtype, int* out) {
  clear_error();
  if (!b || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  switch (dtype) {
    case MX_DTYPE_INT8: case MX_DTYPE_INT16: case MX_DTYPE_INT32: case MX_DTYPE_INT64:
    case MX_DTYPE_UINT8: case MX_DTYPE_UINT16: case MX_DTYPE_UINT32: case MX_DTYPE_UINT64:
    case MX_DTYPE_FLOAT16: case MX_DTYPE_FLOAT32: case MX_DTYPE_FLOAT64: case MX_DTYPE_BFLOAT16:
    case MX_DTYPE_INT4: case MX_DTYPE_UINT4: case MX_DTYPE_BOOL:
      *out = 1;
      break;
    default:
      *out = 0;
  }
  return MX_OK;
}

int mx_backend_synchronize(mx_backend* b) {
  clear_error();
  MX_TRY(check_device(b));
  std::lock_guard<std::recursive_mutex> lk(b->mu);
  MX_CHECK_HIP(wait_stream(b->stream));
  return MX_OK;
}

int mx_backend_set_profiling(mx_backend* b, int enabled) {
  clear_error();
  MX_TRY(check_device(b));
  std::lock_guard<std::recursive_mutex> lk(b->mu);
  b->profiling = enabled != 0;
  return MX_OK;
}

int mx_backend_profile_count(mx_backend* b, int* out) {
  clear_error();
  MX_TRY(check_device(b));
  std::lock_guard<std::recursive_mutex> lk(b->mu);
  MX_TRY(resolve_timings(b));
  *out = (int)b->prof.size();
  return MX_OK;
}

int mx_backend_profile_entry(mx_backend* b, int i, char* name, size_t namelen, int64_t* launches,
                             double* total_ms) {
  clear_error();
  MX_TRY(check_device(b));
  std::lock_guard<std::recursive_mutex> lk(b->mu);
  MX_TRY(resolve_timings(b));
  if (i < 0 || i >= (int)b->prof.size()) return set_error(MX_ERR_INVALID, "profile entry %d out of range", i);
  auto it = b->prof.begin();
  std::advance(it, i);
  copy_str(it->first, name, namelen);
  if (launches) *launches = it->second.launches;
  if (total_ms) *total_ms = it->second.total_ms;
  return MX_OK;
}

int mx_backend_profile_reset(mx_backend* b) {
  clear_error();
  MX_TRY(check_device(b));
  std::lock_guard<std::recursive_mutex> lk(b->mu);
  MX_TRY(resolve_timings(b));
  b->prof.clear();
  return MX_OK;
}

int mx_backend_region_begin(mx_backend* b) {
  clear_error();
  MX_TRY(check_device(b));
  std::lock_guard<std::recursive_mutex> lk(b->mu);
  if (!b->region_start) MX_CHECK_HIP(hipEventCreate(&b->region_start));
  if (!b->region_stop) MX_CHECK_HIP(hipEventCreate(&b->region_stop));
  MX_CHECK_HIP(hipEventRecord(b->region_start, b->stream));
  b->region_open = true;
  return MX_OK;
}

int mx_backend_region_end(mx_backend* b, double* ms) {
  clear_error();
  MX_TRY(check_device(b));
  if (!ms) return set_error(MX_ERR_INVALID, "mx_backend_region_end: ms is NULL");
  std::lock_guard<std::recursive_mutex> lk(b->mu);
  if (!b->region_open) return set_error(MX_ERR_INVALID, "mx_backend_region_end: no region begun");
  b->region_open = false;
  MX_CHECK_HIP(hipEventRecord(b->region_stop, b->stream));
  MX_CHECK_HIP(wait_event(b->region_stop));
  float f = 0.0f;
  MX_CHECK_HIP(hipEventElapsedTime(&f, b->region_start, b->region_stop));
  *ms = f;
  return MX_OK;
}

int mx_backend_debug_fail_alloc_after(mx_backend* b, int n) {
  clear_error();
  if (!b) return set_error(MX_ERR_INVALID, "backend is NULL");
  std::lock_guard<std::recursive_mutex> lk(b->mu);
  b->pool.fail_after = n > 0 ? n : 0;
  return MX_OK;
}

int mx_backend_has_shared_buffers(const mx_backend* b, int* out) {
  clear_error();
  if (!b || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  *out = 0;
  return MX_OK;
}

// ---------------------------------------------------------------------------------------------
// Buffers.
// ---------------------------------------------------------------------------------------------
int mx_buffer_from_flat(mx_backend* b, int device, const void* host, size_t host_nbytes,
                        const mx_shape* shape, mx_buffer** out) {
  clear_error();
  if (!out) return set_error(MX_ERR_INVALID, "out is NULL");
  *out = nullptr;
  MX_TRY(check_device(b));
  if (device != 0) return set_error(MX_ERR_INVALID, "BufferFromFlatData: device %d not available", device);
  Shape s;
  MX_TRY(shape_from_c(shape, &s));
  size_t nb = s.nbytes();
  if (host_nbytes != nb)
    return set_error(MX_ERR_INVALID, "BufferFromFlatData: shape %s needs %zu bytes, got %zu",
                     s.str().c_str(), nb, host_nbytes);
  if (nb && !host) return set_error(MX_ERR_INVALID, "BufferFromFlatData: host data is NULL");
  std::lock_guard<std::recursive_mutex> lk(b->mu);
  void* d = nullptr;
  MX_TRY(dev_alloc(b, nb, &d));
  if (nb) {
    hipError_t e = hipMemcpyAsync(d, host, nb, hipMemcpyHostToDevice, b->stream);
    if (e == hipSuccess) e = wait_stream(b->stream);
    if (e != hipSuccess) {
      dev_free(b, d);
      return set_error(MX_ERR_HIP, "BufferFromFlatData copy failed: %s", hipGetErrorString(e));
    }
  }
  auto* buf = new mx_buffer();
  buf->b = b;
  buf->shape = s;
  buf->dptr = d;
  buf->nbytes = nb;
  b->live_buffers++;
  *out = buf;
  return MX_OK;
}

int mx_buffer_to_flat(mx_buffer* buf, void* host, size_t host_nbytes) {
  clear_error();
  if (!buf) return set_error(MX_ERR_INVALID, "buffer is NULL");
  if (buf->finalized) return set_error(MX_ERR_FINALIZED, "ToFlatData: buffer already finalized");
  MX_TRY(check_device(buf->b));
  if (host_nbytes != buf->nbytes)
    return set_error(MX_ERR_INVALID, "ToFlatData: buffer %s has %zu bytes, destination has %zu",
                     buf->shape.str().c_str(), buf->nbytes, host_nbytes);
  if (buf->nbytes == 0) return MX_OK;
  if (!host) return set_error(MX_ERR_INVALID, "ToFlatData: host is NULL");
  std::lock_guard<std::recursive_mutex> lk(buf->b->mu);
  MX_CHECK_HIP(hipMemcpyAsync(host, buf->dptr, buf->nbytes, hipMemcpyDeviceToHost, buf->b->stream));
  MX_CHECK_HIP(wait_stream(buf->b->stream));
  return MX_OK;
}

int mx_buffer_shape(const mx_buffer* buf, mx_shape* out) {
  clear_error();
  if (!buf || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  if (buf->finalized) return set_error(MX_ERR_FINALIZED, "Shape: buffer already finalized");
  shape_to_c(buf->shape, out);
  return MX_OK;
}

int mx_buffer_device(const mx_buffer* buf, int* out) {
  clear_error();
  if (!buf || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  if (buf->finalized) return set_error(MX_ERR_FINALIZED, "DeviceNum: buffer already finalized");
  *out = 0;
  return MX_OK;
}

int mx_buffer_nbytes(const mx_buffer* buf, size_t* out) {
  clear_error();
  if (!buf || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  if (buf->finalized) return set_error(MX_ERR_FINALIZED, "buffer already finalized");
  *out = buf->nbytes;
  return MX_OK;
}

int mx_buffer_device_ptr(const mx_buffer* buf, void** out) {
  clear_error();
  if (!buf || !out) return set_error(MX_ERR_INVALID, "NULL argument");
  if (buf->finalized) return set_error(MX_ERR_FINALIZED, "buffer already finalized");
  *out = buf->dptr;
  return MX_OK;
}

int mx_buffer_finalize(mx_buffer* buf) {
  clear_error();
  if (!buf) return MX_OK;
  if (buf->finalized) return set_error(MX_ERR_FINALIZED, "Finalize: buffer already finalized");
  mx_backend* b = buf->b;
  {
    std::lock_guard<std::recursive_mutex> lk(b->mu);
    dev_free(b, buf->dptr);
    b->live_buffers--;
  }
  buf->finalized = true;
  buf->dptr = nullptr;
  return MX_OK;
}

int mx_buffer_destroy(mx_buffer* buf) {
  clear_error();
  if (!buf) return MX_OK;
  if (!buf->finalized) MX_TRY(mx_buffer_finalize(buf));
  delete buf;
  return MX_OK;
}

}  // extern "C"
