// Library state: per-thread error text, the registered workspace allocator,
// device properties and dtype promotion.
#include <mutex>
#include <vector>

#include "common.h"

namespace mi {

namespace {
thread_local std::string g_last_error;

mi_alloc_fn g_alloc = nullptr;
mi_free_fn g_free = nullptr;
void* g_alloc_ctx = nullptr;
std::mutex g_alloc_mu;

std::mutex g_cu_mu;
std::vector<int> g_cu_counts;
}  // namespace

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

// Called at the start of every entry point: forgets this thread's previous
// message and any runtime error left by an unrelated earlier HIP call, so
// check_launch reports only the launch it follows.
void clear_error() {
  g_last_error.clear();
  (void)hipGetLastError();
}

mi_status_t check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return MI_ERR_LAUNCH;
  }
  return MI_OK;
}

namespace {
thread_local ScratchArena* t_arena = nullptr;
}

void set_scratch_arena(ScratchArena* arena) { t_arena = arena; }

Workspace::~Workspace() {
  if (ptr_ != nullptr && !from_arena_) {
    mi_free_fn f;
    void* ctx;
    {
      std::lock_guard<std::mutex> g(g_alloc_mu);
      f = g_free;
      ctx = g_alloc_ctx;
    }
    if (f) f(ptr_, (mi_stream_t)stream_, ctx);
  }
}

mi_status_t Workspace::alloc(size_t bytes, hipStream_t stream) {
  if (t_arena != nullptr) {
    ScratchArena& ar = *t_arena;
    const size_t start = (ar.used + 255) & ~(size_t)255;
    if (start > ar.size || bytes > ar.size - start)
      MI_FAIL(MI_ERR_TOO_LARGE,
              "this call needs %zu bytes of scratch (%zu already taken) but the static "
              "scratch holds %zu bytes",
              bytes, start, ar.size);
    ptr_ = ar.base + start;
    ar.used = start + bytes;
    if (ar.used > ar.peak) ar.peak = ar.used;
    stream_ = stream;
    from_arena_ = true;
    return MI_OK;
  }
  mi_alloc_fn a;
  void* ctx;
  {
    std::lock_guard<std::mutex> g(g_alloc_mu);
    a = g_alloc;
    ctx = g_alloc_ctx;
  }
  if (a == nullptr)
    MI_FAIL(MI_ERR_WORKSPACE,
            "a workspace of %zu bytes is needed but no workspace allocator "
            "is registered (mi_set_workspace_allocator)",
            bytes);
  ptr_ = a(bytes == 0 ? 1 : bytes, (mi_stream_t)stream, ctx);
  stream_ = stream;
  if (ptr_ == nullptr)
    MI_FAIL(MI_ERR_WORKSPACE, "workspace allocator returned NULL for %zu bytes",
            bytes);
  return MI_OK;
}

namespace {
std::mutex g_fault_mu;
std::vector<IndexFault*> g_faults;  // per device, host pointers (coherent, mapped)

IndexFault* fault_of(int dev, bool create) {
  std::lock_guard<std::mutex> g(g_fault_mu);
  if ((int)g_faults.size() <= dev) g_faults.resize(dev + 1, nullptr);
  if (g_faults[dev] == nullptr && create) {
    // host allocation is legal inside a stream capture only in relaxed mode
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    (void)hipThreadExchangeStreamCaptureMode(&mode);
    void* p = nullptr;
    const hipError_t e =
        hipHostMalloc(&p, sizeof(IndexFault), hipHostMallocMapped | hipHostMallocCoherent);
    (void)hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    volatile IndexFault* v = static_cast<volatile IndexFault*>(p);
    v->flag = 0;
    v->index = 0;
    v->size = 0;
    g_faults[dev] = static_cast<IndexFault*>(p);
  }
  return g_faults[dev];
}
}  // namespace

IndexFault* index_fault_word() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  IndexFault* h = fault_of(dev, true);
  if (h == nullptr) return nullptr;
  void* d = nullptr;
  if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  return static_cast<IndexFault*>(d);
}

int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> g(g_cu_mu);
  if ((int)g_cu_counts.size() <= dev) g_cu_counts.resize(dev + 1, 0);
  if (g_cu_counts[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
            hipSuccess ||
        n <= 0)
      n = 256;
    g_cu_counts[dev] = n;
  }
  return g_cu_counts[dev];
}

const char* dtype_name(int dt) {
  switch (dt) {
    case MI_U8: return "uint8";
    case MI_I8: return "int8";
    case MI_I16: return "int16";
    case MI_I32: return "int32";
    case MI_I64: return "int64";
    case MI_F16: return "float16";
    case MI_F32: return "float32";
    case MI_F64: return "float64";
    case MI_BOOL: return "bool";
    case MI_BF16: return "bfloat16";
    default: return "unknown";
  }
}

namespace {
int float_rank(int dt) {
  switch (dt) {
    case MI_F16: return 1;
    case MI_BF16: return 1;
    case MI_F32: return 2;
    case MI_F64: return 3;
    default: return 0;
  }
}
int int_width(int dt) {
  switch (dt) {
    case MI_U8: case MI_I8: return 1;
    case MI_I16: return 2;
    case MI_I32: return 4;
    case MI_I64: return 8;
    default: return 0;
  }
}
int signed_of_width(int w) {
  switch (w) {
    case 1: return MI_I8;
    case 2: return MI_I16;
    case 4: return MI_I32;
    default: return MI_I64;
  }
}
}  // namespace

// Same table as c10::promoteTypes restricted to the dtypes of this library.
int promote_types(int a, int b) {
  if (a == b) return a;
  if (a == MI_BOOL) return b;
  if (b == MI_BOOL) return a;
  const bool fa = is_floating(a), fb = is_floating(b);
  if (fa && fb) {
    if ((a == MI_F16 && b == MI_BF16) || (a == MI_BF16 && b == MI_F16)) return MI_F32;
    return float_rank(a) >= float_rank(b) ? a : b;
  }
  if (fa) return a;
  if (fb) return b;
  // both integral
  if (a == MI_U8 || b == MI_U8) {
    const int o = (a == MI_U8) ? b : a;
    // uint8 with a signed type: the signed type at least 16 bits wide
    return int_width(o) < 2 ? MI_I16 : o;
  }
  return signed_of_width(int_width(a) > int_width(b) ? int_width(a) : int_width(b));
}

bool is_contiguous(const mi_tensor_t& t) {
  int64_t expected = 1;
  for (int d = t.ndim - 1; d >= 0; --d) {
    if (t.sizes[d] == 1) continue;
    if (t.strides[d] != expected) return false;
    expected *= t.sizes[d];
  }
  return true;
}

mi_status_t validate(const mi_tensor_t* t, const char* name) {
  if (t == nullptr) MI_FAIL(MI_ERR_INVALID, "%s: descriptor is NULL", name);
  if (t->ndim < 0 || t->ndim > MI_MAX_DIMS)
    MI_FAIL(MI_ERR_INVALID, "%s: ndim %d outside [0, %d]", name, t->ndim,
            MI_MAX_DIMS);
  if (!dtype_valid(t->dtype))
    MI_FAIL(MI_ERR_UNSUPPORTED, "%s: unsupported dtype code %d", name, t->dtype);
  for (int d = 0; d < t->ndim; ++d) {
    if (t->sizes[d] < 0)
      MI_FAIL(MI_ERR_INVALID, "%s: negative size %lld at dim %d", name,
              (long long)t->sizes[d], d);
    if (t->strides[d] < 0)
      MI_FAIL(MI_ERR_UNSUPPORTED, "%s: negative stride at dim %d", name, d);
  }
  if (t->data == nullptr && numel(*t) > 0)
    MI_FAIL(MI_ERR_INVALID, "%s: NULL data with %lld elements", name,
            (long long)numel(*t));
  return MI_OK;
}

}  // namespace mi

extern "C" {

int32_t mi_abi_version(void) { return (1 << 16) | 0; }

const char* mi_last_error(void) { return mi::g_last_error.c_str(); }

mi_status_t mi_set_workspace_allocator(mi_alloc_fn alloc_fn, mi_free_fn free_fn,
                                       void* ctx) {
  if ((alloc_fn == nullptr) != (free_fn == nullptr))
    MI_FAIL(MI_ERR_INVALID, "alloc_fn and free_fn must both be set or both NULL");
  std::lock_guard<std::mutex> g(mi::g_alloc_mu);
  mi::g_alloc = alloc_fn;
  mi::g_free = free_fn;
  mi::g_alloc_ctx = ctx;
  return MI_OK;
}

int32_t mi_device_cu_count(void) { return mi::cu_count(); }

int32_t mi_index_fault_take(int32_t device, int64_t* index, int64_t* dim_size) {
  if (device < 0) return 0;
  mi::IndexFault* f = mi::fault_of(device, false);
  if (f == nullptr) return 0;
  volatile mi::IndexFault* v = f;
  if (v->flag == 0) return 0;
  if (index) *index = v->index;
  if (dim_size) *dim_size = v->size;
  v->flag = 0;
  return 1;
}

}  // extern "C"
