// libmlc_hip.so — the C ABI declared in include/mlc_hip.h.
//
// Host-side HIP runtime for the MI355X backend: code-object modules, the
// arena slab (one hipMalloc, exported to torch through DLPack), pre-resolved
// launch plans, hipGraph capture/replay and hipEvent timing. No exception
// crosses the ABI; failures return a negative code and leave a message.

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "mlc_hip.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& what) {
  g_last_error = what;
  return code;
}

int hip_fail(hipError_t err, const char* what) {
  g_last_error = std::string(what) + ": " + hipGetErrorName(err) + " (" + hipGetErrorString(err) + ")";
  return -static_cast<int>(err);
}

#define MLC_HIP(call)                                   \
  do {                                                  \
    hipError_t _e = (call);                             \
    if (_e != hipSuccess) return hip_fail(_e, #call);   \
  } while (0)

// ---- DLPack ABI (the public DLPack 0.x layout torch accepts as "dltensor")
struct DLDevice {
  int32_t device_type;
  int32_t device_id;
};
struct DLDataType {
  uint8_t code;
  uint8_t bits;
  uint16_t lanes;
};
struct DLTensor {
  void* data;
  DLDevice device;
  int32_t ndim;
  DLDataType dtype;
  int64_t* shape;
  int64_t* strides;
  uint64_t byte_offset;
};
struct DLManagedTensor {
  DLTensor dl_tensor;
  void* manager_ctx;
  void (*deleter)(DLManagedTensor* self);
};
constexpr int32_t kDLROCM = 10;
constexpr uint8_t kDLUInt = 1;

constexpr size_t kErrorWordBytes = 16;

struct Slab {
  void* ptr = nullptr;
  size_t bytes = 0;
  int device = 0;
  std::atomic<int> refs{1};
  // the device's static arena (``scratch``): never freed, never deleted
  bool is_static = false;
};

void slab_release(Slab* s) {
  if (s == nullptr) return;
  if (s->is_static) {
    s->refs.fetch_sub(1);
    return;
  }
  if (s->refs.fetch_sub(1) == 1) {
    if (s->ptr != nullptr) {
      int prev = 0;
      (void)hipGetDevice(&prev);
      (void)hipSetDevice(s->device);
      (void)hipFree(s->ptr);
      (void)hipSetDevice(prev);
    }
    delete s;
  }
}

struct Export {
  DLManagedTensor managed;
  int64_t shape[1];
  int64_t strides[1];
};

void export_deleter(DLManagedTensor* t) {
  Export* e = reinterpret_cast<Export*>(t);
  slab_release(static_cast<Slab*>(t->manager_ctx));
  delete e;
}

struct Entry {
  hipFunction_t fn = nullptr;
  uint32_t grid = 0;
  uint32_t block = 0;
  uint32_t lds = 0;
  std::vector<unsigned char> args;
};

int launch_raw(hipFunction_t fn, uint32_t grid, uint32_t block, uint32_t lds, const void* args,
               size_t size, hipStream_t stream) {
  size_t sz = size;
  void* cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void*>(args),
                 HIP_LAUNCH_PARAM_BUFFER_SIZE, &sz, HIP_LAUNCH_PARAM_END};
  hipError_t e = hipModuleLaunchKernel(fn, grid, 1, 1, block, 1, 1, lds, stream, nullptr, cfg);
  if (e != hipSuccess) return hip_fail(e, "hipModuleLaunchKernel");
  return MLC_OK;
}

// ---- the arena for callers that cannot allocate (mlc_slab_static)
//
// One array per GPU, held from the first context on that GPU until the
// process ends. Its name is a host-side stand-in: the device address comes
// from hipGetSymbolAddress, resolved once per device with that device
// current (in mlc_ctx_create) and kept in g_static[device].
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[MLC_STATIC_SLAB_BYTES];

struct StaticSlab {
  std::once_flag once;
  hipError_t status = hipSuccess;
  Slab slab;
};
StaticSlab g_static[kMaxDevices];

void resolve_static_slab(int device) {
  StaticSlab& st = g_static[device];
  std::call_once(st.once, [&st, device]() {
    void* ptr = nullptr;
    st.status = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (st.status == hipSuccess) {
      st.slab.ptr = ptr;
      st.slab.bytes = MLC_STATIC_SLAB_BYTES;
      st.slab.device = device;
      st.slab.is_static = true;
      st.slab.refs.store(0);
    }
  });
}

}  // namespace

struct mlc_ctx {
  int device = 0;
  Slab* slab = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipStream_t capturing = nullptr;
  // invalid-input word: set by kernels on the device, mirrored into pinned
  // host memory by an asynchronous copy the caller enqueues after its work
  int32_t* err_dev = nullptr;
  volatile int32_t* err_host = nullptr;
};

struct mlc_module {
  hipModule_t mod = nullptr;
  int device = 0;
};

struct mlc_plan {
  mlc_ctx* ctx = nullptr;
  std::vector<Entry> entries;
};

extern "C" {

int mlc_version(void) { return (1 << 16) | 0; }

const char* mlc_last_error(void) { return g_last_error.c_str(); }

int mlc_ctx_create(int device, mlc_ctx** out) {
  if (out == nullptr) return fail(MLC_E_ARG, "mlc_ctx_create: null out");
  int count = 0;
  MLC_HIP(hipGetDeviceCount(&count));
  if (device < 0 || device >= count) return fail(MLC_E_RANGE, "mlc_ctx_create: no such device");
  MLC_HIP(hipSetDevice(device));
  if (device < kMaxDevices) resolve_static_slab(device);
  mlc_ctx* c = new (std::nothrow) mlc_ctx;
  if (c == nullptr) return fail(MLC_E_STATE, "mlc_ctx_create: out of host memory");
  c->device = device;
  *out = c;
  return MLC_OK;
}

int mlc_ctx_destroy(mlc_ctx* ctx) {
  if (ctx == nullptr) return MLC_OK;
  (void)hipSetDevice(ctx->device);
  if (ctx->exec != nullptr) (void)hipGraphExecDestroy(ctx->exec);
  if (ctx->graph != nullptr) (void)hipGraphDestroy(ctx->graph);
  slab_release(ctx->slab);
  if (ctx->err_dev != nullptr) (void)hipFree(ctx->err_dev);
  if (ctx->err_host != nullptr) (void)hipHostFree(const_cast<int32_t*>(ctx->err_host));
  delete ctx;
  return MLC_OK;
}

int mlc_module_load(mlc_ctx* ctx, const void* image, size_t size, mlc_module** out) {
  if (ctx == nullptr || image == nullptr || size == 0 || out == nullptr)
    return fail(MLC_E_ARG, "mlc_module_load: bad argument");
  MLC_HIP(hipSetDevice(ctx->device));
  hipModule_t m = nullptr;
  MLC_HIP(hipModuleLoadData(&m, image));
  mlc_module* w = new (std::nothrow) mlc_module;
  if (w == nullptr) {
    (void)hipModuleUnload(m);
    return fail(MLC_E_STATE, "mlc_module_load: out of host memory");
  }
  w->mod = m;
  w->device = ctx->device;
  *out = w;
  return MLC_OK;
}

int mlc_module_unload(mlc_module* mod) {
  if (mod == nullptr) return MLC_OK;
  (void)hipSetDevice(mod->device);
  hipError_t e = hipModuleUnload(mod->mod);
  delete mod;
  if (e != hipSuccess) return hip_fail(e, "hipModuleUnload");
  return MLC_OK;
}

int mlc_function(mlc_module* mod, const char* name, mlc_fn* out) {
  if (mod == nullptr || name == nullptr || out == nullptr)
    return fail(MLC_E_ARG, "mlc_function: bad argument");
  hipFunction_t f = nullptr;
  hipError_t e = hipModuleGetFunction(&f, mod->mod, name);
  if (e != hipSuccess) return hip_fail(e, (std::string("hipModuleGetFunction ") + name).c_str());
  *out = reinterpret_cast<mlc_fn>(f);
  return MLC_OK;
}

int mlc_slab_alloc(mlc_ctx* ctx, size_t bytes, void** dptr) {
  if (ctx == nullptr || dptr == nullptr) return fail(MLC_E_ARG, "mlc_slab_alloc: bad argument");
  if (bytes == 0) bytes = 256;
  if (ctx->slab != nullptr && ctx->slab->bytes >= bytes) {
    *dptr = ctx->slab->ptr;
    return MLC_OK;
  }
  if (ctx->slab != nullptr && ctx->slab->is_static)
    return fail(MLC_E_STATE, "mlc_slab_alloc: the context's arena is the static one");
  if (ctx->slab != nullptr && ctx->slab->refs.load() > 1)
    return fail(MLC_E_STATE, "mlc_slab_alloc: cannot grow a slab that is still exported");
  MLC_HIP(hipSetDevice(ctx->device));
  void* p = nullptr;
  MLC_HIP(hipMalloc(&p, bytes));
  slab_release(ctx->slab);
  Slab* s = new (std::nothrow) Slab;
  if (s == nullptr) {
    (void)hipFree(p);
    return fail(MLC_E_STATE, "mlc_slab_alloc: out of host memory");
  }
  s->ptr = p;
  s->bytes = bytes;
  s->device = ctx->device;
  ctx->slab = s;
  *dptr = p;
  return MLC_OK;
}

int mlc_slab_static(mlc_ctx* ctx, size_t bytes, void** dptr) {
  if (ctx == nullptr || dptr == nullptr) return fail(MLC_E_ARG, "mlc_slab_static: bad argument");
  if (bytes > MLC_STATIC_SLAB_BYTES)
    return fail(MLC_E_RANGE, "mlc_slab_static: " + std::to_string(bytes) +
                                 " bytes requested, the static arena holds " +
                                 std::to_string(static_cast<size_t>(MLC_STATIC_SLAB_BYTES)));
  if (ctx->device >= kMaxDevices)
    return fail(MLC_E_RANGE, "mlc_slab_static: device index beyond the static arena table");
  StaticSlab& st = g_static[ctx->device];
  if (st.status != hipSuccess) return hip_fail(st.status, "mlc_slab_static: hipGetSymbolAddress");
  if (st.slab.ptr == nullptr) return fail(MLC_E_STATE, "mlc_slab_static: static arena unresolved");
  if (ctx->slab == &st.slab) {
    *dptr = st.slab.ptr;
    return MLC_OK;
  }
  if (ctx->slab != nullptr)
    return fail(MLC_E_STATE,
                "mlc_slab_static: the context already owns an allocated slab (freeing it "
                "would call hipFree)");
  st.slab.refs.fetch_add(1);
  ctx->slab = &st.slab;
  *dptr = st.slab.ptr;
  return MLC_OK;
}

int mlc_slab_dlpack(mlc_ctx* ctx, void** managed_tensor) {
  if (ctx == nullptr || managed_tensor == nullptr)
    return fail(MLC_E_ARG, "mlc_slab_dlpack: bad argument");
  if (ctx->slab == nullptr) return fail(MLC_E_STATE, "mlc_slab_dlpack: no slab allocated");
  Export* e = new (std::nothrow) Export;
  if (e == nullptr) return fail(MLC_E_STATE, "mlc_slab_dlpack: out of host memory");
  Slab* s = ctx->slab;
  s->refs.fetch_add(1);
  e->shape[0] = static_cast<int64_t>(s->bytes);
  e->strides[0] = 1;
  DLTensor& t = e->managed.dl_tensor;
  t.data = s->ptr;
  t.device = DLDevice{kDLROCM, ctx->device};
  t.ndim = 1;
  t.dtype = DLDataType{kDLUInt, 8, 1};
  t.shape = e->shape;
  t.strides = e->strides;
  t.byte_offset = 0;
  e->managed.manager_ctx = s;
  e->managed.deleter = export_deleter;
  *managed_tensor = &e->managed;
  return MLC_OK;
}

int mlc_launch(mlc_fn fn, uint32_t grid, uint32_t block, uint32_t lds_bytes, const void* kernarg,
               size_t size, void* stream) {
  if (fn == nullptr || grid == 0 || block == 0 || block > 1024)
    return fail(MLC_E_ARG, "mlc_launch: bad launch geometry");
  return launch_raw(reinterpret_cast<hipFunction_t>(fn), grid, block, lds_bytes, kernarg, size,
                    static_cast<hipStream_t>(stream));
}

int mlc_plan_create(mlc_ctx* ctx, int n_entries, mlc_plan** out) {
  if (ctx == nullptr || n_entries < 0 || out == nullptr)
    return fail(MLC_E_ARG, "mlc_plan_create: bad argument");
  mlc_plan* p = new (std::nothrow) mlc_plan;
  if (p == nullptr) return fail(MLC_E_STATE, "mlc_plan_create: out of host memory");
  p->ctx = ctx;
  p->entries.resize(static_cast<size_t>(n_entries));
  *out = p;
  return MLC_OK;
}

int mlc_plan_set(mlc_plan* plan, int index, mlc_fn fn, uint32_t grid, uint32_t block,
                 uint32_t lds_bytes, const void* kernarg, size_t size) {
  if (plan == nullptr || fn == nullptr) return fail(MLC_E_ARG, "mlc_plan_set: bad argument");
  if (index < 0 || static_cast<size_t>(index) >= plan->entries.size())
    return fail(MLC_E_RANGE, "mlc_plan_set: index out of range");
  if (grid == 0 || block == 0 || block > 1024)
    return fail(MLC_E_ARG, "mlc_plan_set: bad launch geometry");
  Entry& e = plan->entries[static_cast<size_t>(index)];
  e.fn = reinterpret_cast<hipFunction_t>(fn);
  e.grid = grid;
  e.block = block;
  e.lds = lds_bytes;
  const unsigned char* b = static_cast<const unsigned char*>(kernarg);
  e.args.assign(b, b + size);
  return MLC_OK;
}

int mlc_plan_run(mlc_plan* plan, int begin, int end, void* stream) {
  if (plan == nullptr) return fail(MLC_E_ARG, "mlc_plan_run: null plan");
  if (begin < 0 || end < begin || static_cast<size_t>(end) > plan->entries.size())
    return fail(MLC_E_RANGE, "mlc_plan_run: range out of bounds");
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int i = begin; i < end; ++i) {
    const Entry& e = plan->entries[static_cast<size_t>(i)];
    if (e.fn == nullptr) return fail(MLC_E_STATE, "mlc_plan_run: entry was never set");
    int rc = launch_raw(e.fn, e.grid, e.block, e.lds, e.args.data(), e.args.size(), s);
    if (rc != MLC_OK) return rc;
  }
  return MLC_OK;
}

int mlc_plan_destroy(mlc_plan* plan) {
  delete plan;
  return MLC_OK;
}

int mlc_graph_begin(mlc_ctx* ctx, void* stream) {
  if (ctx == nullptr || stream == nullptr) return fail(MLC_E_ARG, "mlc_graph_begin: bad argument");
  if (ctx->capturing != nullptr) return fail(MLC_E_STATE, "mlc_graph_begin: already capturing");
  MLC_HIP(hipSetDevice(ctx->device));
  MLC_HIP(hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal));
  ctx->capturing = static_cast<hipStream_t>(stream);
  return MLC_OK;
}

int mlc_graph_end(mlc_ctx* ctx) {
  if (ctx == nullptr) return fail(MLC_E_ARG, "mlc_graph_end: null ctx");
  if (ctx->capturing == nullptr) return fail(MLC_E_STATE, "mlc_graph_end: not capturing");
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(ctx->capturing, &g);
  ctx->capturing = nullptr;
  if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
  hipGraphExec_t x = nullptr;
  e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    return hip_fail(e, "hipGraphInstantiate");
  }
  if (ctx->exec != nullptr) (void)hipGraphExecDestroy(ctx->exec);
  if (ctx->graph != nullptr) (void)hipGraphDestroy(ctx->graph);
  ctx->graph = g;
  ctx->exec = x;
  return MLC_OK;
}

int mlc_graph_replay(mlc_ctx* ctx, void* stream) {
  if (ctx == nullptr) return fail(MLC_E_ARG, "mlc_graph_replay: null ctx");
  if (ctx->exec == nullptr) return fail(MLC_E_STATE, "mlc_graph_replay: nothing captured");
  MLC_HIP(hipGraphLaunch(ctx->exec, static_cast<hipStream_t>(stream)));
  return MLC_OK;
}

int mlc_graph_node_count(mlc_ctx* ctx, size_t* out) {
  if (ctx == nullptr || out == nullptr) return fail(MLC_E_ARG, "mlc_graph_node_count: bad argument");
  if (ctx->graph == nullptr) return fail(MLC_E_STATE, "mlc_graph_node_count: nothing captured");
  size_t n = 0;
  MLC_HIP(hipGraphGetNodes(ctx->graph, nullptr, &n));
  *out = n;
  return MLC_OK;
}

int mlc_time_entry(mlc_plan* plan, int index, int iters, void* stream, float* ms_out) {
  if (plan == nullptr || ms_out == nullptr || iters <= 0)
    return fail(MLC_E_ARG, "mlc_time_entry: bad argument");
  if (index < 0 || static_cast<size_t>(index) >= plan->entries.size())
    return fail(MLC_E_RANGE, "mlc_time_entry: index out of range");
  const Entry& e = plan->entries[static_cast<size_t>(index)];
  if (e.fn == nullptr) return fail(MLC_E_STATE, "mlc_time_entry: entry was never set");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipEvent_t start = nullptr, stop = nullptr;
  MLC_HIP(hipEventCreate(&start));
  hipError_t err = hipEventCreate(&stop);
  if (err != hipSuccess) {
    (void)hipEventDestroy(start);
    return hip_fail(err, "hipEventCreate");
  }
  int rc = MLC_OK;
  float ms = 0.0f;
  err = hipEventRecord(start, s);
  for (int i = 0; err == hipSuccess && rc == MLC_OK && i < iters; ++i)
    rc = launch_raw(e.fn, e.grid, e.block, e.lds, e.args.data(), e.args.size(), s);
  if (err == hipSuccess && rc == MLC_OK) err = hipEventRecord(stop, s);
  if (err == hipSuccess && rc == MLC_OK) err = hipEventSynchronize(stop);
  if (err == hipSuccess && rc == MLC_OK) err = hipEventElapsedTime(&ms, start, stop);
  (void)hipEventDestroy(start);
  (void)hipEventDestroy(stop);
  if (rc != MLC_OK) return rc;
  if (err != hipSuccess) return hip_fail(err, "mlc_time_entry");
  *ms_out = ms / static_cast<float>(iters);
  return MLC_OK;
}

int mlc_error_word(mlc_ctx* ctx, void** device_word) {
  if (ctx == nullptr || device_word == nullptr) return fail(MLC_E_ARG, "mlc_error_word: bad argument");
  if (ctx->err_dev == nullptr) {
    MLC_HIP(hipSetDevice(ctx->device));
    void* d = nullptr;
    void* h = nullptr;
    MLC_HIP(hipMalloc(&d, kErrorWordBytes));
    hipError_t e = hipHostMalloc(&h, kErrorWordBytes, hipHostMallocDefault);
    if (e == hipSuccess) e = hipMemset(d, 0, kErrorWordBytes);
    if (e != hipSuccess) {
      (void)hipFree(d);
      if (h != nullptr) (void)hipHostFree(h);
      return hip_fail(e, "mlc_error_word");
    }
    std::memset(h, 0, kErrorWordBytes);
    ctx->err_dev = static_cast<int32_t*>(d);
    ctx->err_host = static_cast<volatile int32_t*>(h);
  }
  *device_word = ctx->err_dev;
  return MLC_OK;
}

int mlc_error_fetch(mlc_ctx* ctx, void* stream) {
  if (ctx == nullptr) return fail(MLC_E_ARG, "mlc_error_fetch: null ctx");
  if (ctx->err_dev == nullptr) return fail(MLC_E_STATE, "mlc_error_fetch: no error word");
  MLC_HIP(hipMemcpyAsync(const_cast<int32_t*>(ctx->err_host), ctx->err_dev, kErrorWordBytes,
                         hipMemcpyDeviceToHost, static_cast<hipStream_t>(stream)));
  return MLC_OK;
}

int mlc_error_poll(mlc_ctx* ctx, int32_t* value) {
  if (ctx == nullptr || value == nullptr) return fail(MLC_E_ARG, "mlc_error_poll: bad argument");
  *value = ctx->err_host == nullptr ? 0 : ctx->err_host[0];
  return MLC_OK;
}

int mlc_error_clear(mlc_ctx* ctx) {
  if (ctx == nullptr) return fail(MLC_E_ARG, "mlc_error_clear: null ctx");
  if (ctx->err_dev == nullptr) return MLC_OK;
  MLC_HIP(hipSetDevice(ctx->device));
  MLC_HIP(hipDeviceSynchronize());
  MLC_HIP(hipMemset(ctx->err_dev, 0, kErrorWordBytes));
  for (size_t i = 0; i < kErrorWordBytes / sizeof(int32_t); ++i) ctx->err_host[i] = 0;
  return MLC_OK;
}

int mlc_device_synchronize(mlc_ctx* ctx) {
  if (ctx == nullptr) return fail(MLC_E_ARG, "mlc_device_synchronize: null ctx");
  MLC_HIP(hipSetDevice(ctx->device));
  MLC_HIP(hipDeviceSynchronize());
  return MLC_OK;
}

}  // extern "C"
