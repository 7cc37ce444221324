// Runtime behind the PJRT handles (see runtime.h). Host ↔ device crossings follow the reference's call contracts:
//   BufferFromHostBuffer consumes host bytes before returning (kImmutableOnlyDuringCall, buffers.rs:1875-1883);
//   ToHostBuffer completes through its event (buffers.rs:1237-1266); Execute returns one done event per device and
//   one buffer per output (programs.rs:923-962).
#include "runtime.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <set>
#include <sstream>
#include <thread>
#include <vector>

#include "kernels/kernels.h"

namespace ryft {

hipEvent_t& pending_start() {
  static thread_local hipEvent_t e = nullptr;
  return e;
}


// ------------------------------------------------------------------------------------------------ events
EventState::~EventState() {
  if (hip_event) (void)hipEventDestroy(hip_event);
}

void EventState::set_ready(PJRT_Error_Code c, const std::string& msg) {
  std::vector<std::pair<PJRT_Event_OnReadyCallback, void*>> cbs;
  {
    std::lock_guard<std::mutex> lk(mu);
    if (ready) return;
    if (poisoned) c = code;  // the poison's error wins over the device work's own outcome
    if (c == PJRT_Error_Code_OK && on_complete) {
      try {
        on_complete();
      } catch (const std::exception& e) {
        c = PJRT_Error_Code_INTERNAL;
        message = e.what();
      }
    }
    on_complete = nullptr;
    ready = true;
    code = c;
    if (c != PJRT_Error_Code_OK && message.empty()) message = msg;
    cbs.swap(callbacks);
  }
  cv.notify_all();
  for (auto& cb : cbs)
    cb.first(code == PJRT_Error_Code_OK ? nullptr : make_pjrt_error(code, message, payload), cb.second);
}

bool EventState::error_now(Status* out) {
  std::lock_guard<std::mutex> lk(mu);
  if (!(ready || poisoned) || code == PJRT_Error_Code_OK) return false;
  *out = Status(code, message, payload);
  return true;
}

bool EventState::poison(const Status& err) {
  std::lock_guard<std::mutex> lk(mu);
  if (ready || poisoned) return false;
  poisoned = true;
  code = err.code;
  message = err.what();
  payload = err.payload;
  return true;
}

EventPtr error_event(const Status& err) {
  auto e = std::make_shared<EventState>();
  e->payload = err.payload;
  e->set_ready(err.code, err.what());
  return e;
}

void EventState::wait() {
  {
    std::lock_guard<std::mutex> lk(mu);
    if (ready) return;
  }
  if (hip_event) {
    hipError_t e = hipEventSynchronize(hip_event);
    if (e == hipSuccess) set_ready(PJRT_Error_Code_OK, "");
    else set_ready(PJRT_Error_Code_INTERNAL, std::string("device execution failed: ") + hipGetErrorString(e));
    return;
  }
  std::unique_lock<std::mutex> lk(mu);
  cv.wait(lk, [&] { return ready; });
}

bool EventState::poll() {
  {
    std::lock_guard<std::mutex> lk(mu);
    if (ready) return true;
  }
  if (!hip_event) return false;
  hipError_t e = hipEventQuery(hip_event);
  if (e == hipErrorNotReady) return false;
  if (e == hipSuccess) set_ready(PJRT_Error_Code_OK, "");
  else set_ready(PJRT_Error_Code_INTERNAL, std::string("device execution failed: ") + hipGetErrorString(e));
  return true;
}

// ------------------------------------------------------------------------------------------------ allocator
DeviceAllocator::~DeviceAllocator() {
  std::lock_guard<std::mutex> lk(mu_);
  for (auto& kv : free_)
    for (void* p : kv.second) (void)hipFree(p);
  free_.clear();
}

size_t DeviceAllocator::round_size(size_t bytes) {
  if (bytes < 256) return 256;
  if (bytes <= (1u << 20)) {
    size_t s = 256;
    while (s < bytes) s <<= 1;
    return s;
  }
  const size_t g = 2u << 20;
  return (bytes + g - 1) / g * g;
}

void DeviceAllocator::trim() {
  for (auto& kv : free_)
    for (void* p : kv.second) (void)hipFree(p);
  free_.clear();
}

void* DeviceAllocator::allocate(size_t bytes) {
  size_t sz = round_size(bytes);
  std::lock_guard<std::mutex> lk(mu_);
  void* p = nullptr;
  auto it = free_.find(sz);
  if (it != free_.end() && !it->second.empty()) {
    p = it->second.back();
    it->second.pop_back();
  } else {
    HIP_CHECK(hipSetDevice(device_));
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      trim();
      e = hipMalloc(&p, sz);
      if (e != hipSuccess) {
        (void)hipGetLastError();
        fail(PJRT_Error_Code_RESOURCE_EXHAUSTED, "out of device memory allocating " + std::to_string(sz) + " bytes");
      }
    }
    ++allocs_;
  }
  live_[p] = sz;
  in_use_ += (int64_t)sz;
  peak_ = std::max(peak_, in_use_);
  return p;
}

void DeviceAllocator::release(void* p) {
  // Every use of device memory is ordered on the device's single stream, so a block released here can be handed to
  // the next allocation immediately: that allocation's work is enqueued after every pending use of the block.
  std::lock_guard<std::mutex> lk(mu_);
  auto it = live_.find(p);
  if (it == live_.end()) return;
  free_[it->second].push_back(p);
  in_use_ -= (int64_t)it->second;
  live_.erase(it);
}

PinnedPool::~PinnedPool() {
  for (auto& c : chunks_) {
    if (c->last_use) (void)hipEventDestroy(c->last_use);
    if (c->ptr) (void)hipHostFree(c->ptr);
  }
}

PinnedPool::Chunk* PinnedPool::acquire(size_t bytes) {
  std::lock_guard<std::mutex> lk(mu_);
  bytes = std::max<size_t>(bytes, 1);
  for (auto& c : chunks_) {
    if (c->busy || c->bytes < bytes || c->bytes > 4 * bytes + (1u << 20)) continue;
    if (c->last_use && hipEventQuery(c->last_use) != hipSuccess) continue;
    c->busy = true;
    return c.get();
  }
  auto c = std::make_unique<Chunk>();
  size_t sz = (bytes + (1u << 20) - 1) & ~((size_t)(1u << 20) - 1);
  HIP_CHECK(hipHostMalloc(&c->ptr, sz, hipHostMallocDefault));
  c->bytes = sz;
  HIP_CHECK(hipEventCreateWithFlags(&c->last_use, hipEventDisableTiming));
  c->busy = true;
  chunks_.push_back(std::move(c));
  return chunks_.back().get();
}

void PinnedPool::release(Chunk* c, hipStream_t stream) {
  std::lock_guard<std::mutex> lk(mu_);
  (void)hipEventRecord(c->last_use, stream);
  c->busy = false;
}

void PinnedPool::release_now(Chunk* c) {
  std::lock_guard<std::mutex> lk(mu_);
  c->busy = false;
}

// ------------------------------------------------------------------------------------------------ client
static void register_live_client(Client* c);

Client::Client(const std::vector<int>& visible, bool compile_only) {
  if (compile_only) {
    // no device is touched: programs compile to plans (inspectable through the extension) but cannot execute
    platform_version = "ryft-mi355x 0.1 (compile-only)";
    return;
  }
  int count = 0;
  HIP_CHECK(hipGetDeviceCount(&count));
  if (count == 0) fail(PJRT_Error_Code_FAILED_PRECONDITION, "no HIP devices are visible");
  std::vector<int> ords = visible;
  if (ords.empty())
    for (int i = 0; i < count; ++i) ords.push_back(i);
  int rt = 0;
  (void)hipRuntimeGetVersion(&rt);
  platform_version = "ryft-mi355x 0.1 (HIP runtime " + std::to_string(rt) + ", gfx950)";
  for (size_t i = 0; i < ords.size(); ++i) {
    int o = ords[i];
    if (o < 0 || o >= count) invalid("visible device " + std::to_string(o) + " does not exist");
    hipDeviceProp_t prop;
    HIP_CHECK(hipGetDeviceProperties(&prop, o));
    std::string arch = prop.gcnArchName;
    if (arch.rfind("gfx950", 0) != 0)
      fail(PJRT_Error_Code_FAILED_PRECONDITION,
           "device " + std::to_string(o) + " is " + arch + "; this plugin's kernels are built for gfx950 (MI355X)");
    auto d = std::make_unique<Device>();
    d->client = this;
    d->id = (int)i;
    d->hip_ordinal = o;
    d->arch = arch;
    d->kind = std::string(prop.name[0] ? prop.name : "AMD Instinct MI355X");
    d->debug = "MI355X:" + std::to_string(i);
    d->to_string = "MI355XDevice(id=" + std::to_string(i) + ", arch=" + arch + ")";
    d->attribute_strings = {"device_vendor", "AMD", "gfx_arch", arch, "core_count"};
    HIP_CHECK(hipSetDevice(o));
    HIP_CHECK(hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking));
    (void)noalloc_scratch(o);  // set-up of the allocation-free entry point on this device (retried on its first call)
    d->allocator = std::make_unique<DeviceAllocator>(o);
    auto m = std::make_unique<Memory>();
    m->client = this;
    m->id = (int)i;
    m->debug = "MI355X_HBM:" + std::to_string(i);
    m->to_string = "MemorySpace(kind=device, id=" + std::to_string(i) + ")";
    m->devices.push_back(d.get());
    d->memories.push_back(m.get());
    d->default_memory = m.get();
    int cus = prop.multiProcessorCount;
    auto mk = [](const std::string& name, const std::string& val) {
      PJRT_NamedValue v{};
      v.struct_size = sizeof(PJRT_NamedValue);
      v.name = name.c_str();
      v.name_size = name.size();
      v.type = PJRT_NamedValue_kString;
      v.string_value = val.c_str();
      v.value_size = val.size();
      return v;
    };
    d->attributes.push_back(mk(d->attribute_strings[0], d->attribute_strings[1]));
    d->attributes.push_back(mk(d->attribute_strings[2], d->attribute_strings[3]));
    PJRT_NamedValue cv{};
    cv.struct_size = sizeof(PJRT_NamedValue);
    cv.name = d->attribute_strings[4].c_str();
    cv.name_size = d->attribute_strings[4].size();
    cv.type = PJRT_NamedValue_kInt64;
    cv.int64_value = cus;
    cv.value_size = 1;
    d->attributes.push_back(cv);
    device_ptrs.push_back(d.get());
    memory_ptrs.push_back(m.get());
    devices.push_back(std::move(d));
    memories.push_back(std::move(m));
  }
  worker = std::thread([this] {
    for (;;) {
      EventPtr e;
      {
        std::unique_lock<std::mutex> lk(q_mu);
        q_cv.wait(lk, [&] { return stopping || !queue.empty(); });
        if (queue.empty()) return;
        e = queue.front();
        queue.pop_front();
      }
      e->wait();
    }
  });
  register_live_client(this);
}

// Clients alive in this process. A host that exits without destroying its clients (a garbage-collected
// wrapper whose finalizer never ran, for one) would leave each client's completion worker running, possibly
// inside a HIP call, while the HIP runtime tears itself down at exit. The exit hook below is registered after the
// first client has initialised HIP, so it runs before the runtime's own exit-time teardown: it stops every live
// client's worker and drains its streams.
static std::mutex& live_clients_mu() {
  static std::mutex m;
  return m;
}
static std::set<Client*>& live_clients() {
  static std::set<Client*> s;
  return s;
}
static void quiesce_live_clients() {
  std::lock_guard<std::mutex> lk(live_clients_mu());
  for (Client* c : live_clients()) c->stop_worker();
}
static void register_live_client(Client* c) {
  static std::once_flag hook;
  std::lock_guard<std::mutex> lk(live_clients_mu());  // constructs the registry before the hook is registered
  live_clients().insert(c);
  std::call_once(hook, [] { std::atexit(quiesce_live_clients); });
}

void Client::stop_worker() {
  {
    std::lock_guard<std::mutex> lk(q_mu);
    stopping = true;
  }
  q_cv.notify_all();
  if (worker.joinable()) worker.join();
  for (auto& d : devices) {
    (void)hipSetDevice(d->hip_ordinal);
    (void)hipStreamSynchronize(d->stream);
  }
}

Client::~Client() {
  {
    std::lock_guard<std::mutex> lk(live_clients_mu());
    live_clients().erase(this);
  }
  stop_worker();
  {
    std::lock_guard<std::mutex> lk(prof_mu);
    timings.clear();
  }
  for (auto& d : devices) {
    d->allocator.reset();
    (void)hipStreamDestroy(d->stream);
  }
}

void Client::enqueue_completion(const EventPtr& e) {
  {
    std::lock_guard<std::mutex> lk(q_mu);
    queue.push_back(e);
  }
  q_cv.notify_one();
}

EventPtr Client::record_event(Device* d, std::function<void()> on_complete) {
  auto e = std::make_shared<EventState>();
  HIP_CHECK(hipEventCreateWithFlags(&e->hip_event, hipEventDisableTiming));
  HIP_CHECK(hipEventRecord(e->hip_event, d->stream));
  e->on_complete = std::move(on_complete);
  enqueue_completion(e);
  return e;
}

std::shared_ptr<DeviceMem> Client::allocate(Device* d, size_t bytes) {
  auto m = std::make_shared<DeviceMem>();
  m->ptr = d->allocator->allocate(bytes);
  m->bytes = bytes;
  m->alloc = d->allocator.get();
  return m;
}

static EventPtr ready_event() {
  auto e = std::make_shared<EventState>();
  e->ready = true;
  return e;
}

// ------------------------------------------------------------------------------------------------ transfers
// Host memcpy between pageable and pinned memory, split over a few threads for large copies (one thread moves
// ~5-10 GB/s; the PCIe transfer behind it several times that).
static void host_copy(void* dst, const void* src, size_t bytes) {
  constexpr size_t kSplit = (size_t)8 << 20;
  const unsigned hw = std::thread::hardware_concurrency();
  const size_t nt = std::min<size_t>({bytes / kSplit, 8, hw ? hw : 1});
  if (nt < 2) {
    memcpy(dst, src, bytes);
    return;
  }
  // pieces of ceil(bytes / nt) rounded up to a page: nt of them always cover the whole buffer
  const size_t piece = ((bytes + nt - 1) / nt + 4095) & ~(size_t)4095;
  std::vector<std::thread> pool;
  for (size_t i = 1; i < nt; ++i) {
    const size_t off = i * piece;
    if (off >= bytes) break;
    const size_t n = std::min(piece, bytes - off);
    try {
      pool.emplace_back([=] { memcpy((char*)dst + off, (const char*)src + off, n); });
    } catch (...) {  // no thread to be had: the calling thread copies the rest
      memcpy((char*)dst + off, (const char*)src + off, bytes - off);
      break;
    }
  }
  memcpy(dst, src, std::min(piece, bytes));
  for (auto& th : pool) th.join();
}

Buffer* buffer_from_host(Client* c, Device* d, const void* data, DType t, const std::vector<int64_t>& dims,
                         const int64_t* byte_strides, size_t num_byte_strides, EventPtr* done_with_host) {
  for (auto x : dims)
    if (x < 0) invalid("negative dimension in buffer shape " + shape_str(dims));
  auto b = std::make_unique<Buffer>();
  b->client = c;
  b->device = d;
  b->dtype = t;
  b->dims = dims;
  for (int i = (int)dims.size() - 1; i >= 0; --i) b->minor_to_major.push_back(i);
  size_t bytes = b->bytes();
  b->mem = c->allocate(d, bytes);
  const void* src = data;
  std::vector<uint8_t> gathered;
  if (byte_strides && num_byte_strides) {
    if (num_byte_strides != dims.size()) invalid("byte_strides must have one entry per dimension");
    // dense row-major strides need no gather
    int64_t expect = (int64_t)dtype_size(t);
    bool dense = true;
    for (int i = (int)dims.size() - 1; i >= 0; --i) {
      if (dims[i] != 1 && byte_strides[i] != expect) dense = false;
      expect *= dims[i];
    }
    if (!dense) {
      gathered.resize(bytes);
      size_t es = dtype_size(t);
      int64_t n = num_elements(dims);
      std::vector<int64_t> idx(dims.size(), 0);
      for (int64_t i = 0; i < n; ++i) {
        int64_t off = 0;
        for (size_t k = 0; k < dims.size(); ++k) off += idx[k] * byte_strides[k];
        memcpy(gathered.data() + i * es, (const uint8_t*)data + off, es);
        for (int k = (int)dims.size() - 1; k >= 0; --k) {
          if (++idx[k] < dims[k]) break;
          idx[k] = 0;
        }
      }
      src = gathered.data();
    }
  }
  if (bytes > 0 && !src) invalid("BufferFromHostBuffer: data is null");
  {
    std::lock_guard<std::recursive_mutex> lk(d->launch_mu);
    HIP_CHECK(hipSetDevice(d->hip_ordinal));
    if (bytes > 0) {
      auto* chunk = c->pinned.acquire(bytes);
      host_copy(chunk->ptr, src, bytes);
      hipError_t e = hipMemcpyAsync(b->mem->ptr, chunk->ptr, bytes, hipMemcpyHostToDevice, d->stream);
      c->pinned.release(chunk, d->stream);
      if (e != hipSuccess) fail(PJRT_Error_Code_INTERNAL, std::string("host-to-device copy failed: ") + hipGetErrorString(e));
    }
    b->ready = c->record_event(d);
  }
  if (done_with_host) *done_with_host = ready_event();  // host bytes were consumed before returning
  return b.release();
}

// The error `b` carries (an error buffer, or the result of a poisoned execution), if any.
static bool buffer_error(const Buffer* b, Status* err) { return b->ready && b->ready->error_now(err); }

EventPtr buffer_to_host(Buffer* b, void* dst, size_t dst_size) {
  if (b->deleted) fail(PJRT_Error_Code_FAILED_PRECONDITION, "ToHostBuffer on a deleted buffer");
  size_t bytes = b->bytes();
  if (dst_size < bytes) invalid("ToHostBuffer: destination holds " + std::to_string(dst_size) + " bytes, need " + std::to_string(bytes));
  Status err(PJRT_Error_Code_OK, "");
  if (buffer_error(b, &err)) return error_event(err);
  Client* c = b->client;
  Device* d = b->device;
  if (bytes == 0) return ready_event();
  std::lock_guard<std::recursive_mutex> lk(d->launch_mu);
  HIP_CHECK(hipSetDevice(d->hip_ordinal));
  auto* chunk = c->pinned.acquire(bytes);
  hipError_t e = hipMemcpyAsync(chunk->ptr, b->mem->ptr, bytes, hipMemcpyDeviceToHost, d->stream);
  if (e != hipSuccess) {
    c->pinned.release_now(chunk);
    fail(PJRT_Error_Code_INTERNAL, std::string("device-to-host copy failed: ") + hipGetErrorString(e));
  }
  auto mem = b->mem;  // keep the source alive until the copy completes
  PinnedPool* pool = &c->pinned;
  return c->record_event(d, [chunk, dst, bytes, mem, pool] {
    host_copy(dst, chunk->ptr, bytes);
    pool->release_now(chunk);
  });
}

EventPtr buffer_raw_to_host(Buffer* b, void* dst, int64_t offset, int64_t size) {
  if (b->deleted) fail(PJRT_Error_Code_FAILED_PRECONDITION, "CopyRawToHost on a deleted buffer");
  const int64_t bytes = (int64_t)b->bytes();
  if (offset < 0 || size < 0 || offset > bytes || size > bytes - offset)
    invalid("CopyRawToHost: bytes [" + std::to_string(offset) + ", " + std::to_string(offset) + " + " +
            std::to_string(size) + ") are outside the buffer's " + std::to_string(bytes) + " bytes");
  if (size > 0 && !dst) invalid("CopyRawToHost: dst is null");
  Status err(PJRT_Error_Code_OK, "");
  if (buffer_error(b, &err)) return error_event(err);
  Client* c = b->client;
  Device* d = b->device;
  if (size == 0) return ready_event();
  std::lock_guard<std::recursive_mutex> lk(d->launch_mu);
  HIP_CHECK(hipSetDevice(d->hip_ordinal));
  auto* chunk = c->pinned.acquire((size_t)size);
  hipError_t e = hipMemcpyAsync(chunk->ptr, (const char*)b->mem->ptr + offset, (size_t)size, hipMemcpyDeviceToHost,
                                d->stream);
  if (e != hipSuccess) {
    c->pinned.release_now(chunk);
    fail(PJRT_Error_Code_INTERNAL, std::string("device-to-host copy failed: ") + hipGetErrorString(e));
  }
  auto mem = b->mem;  // keep the source alive until the copy completes
  PinnedPool* pool = &c->pinned;
  return c->record_event(d, [chunk, dst, size, mem, pool] {
    memcpy(dst, chunk->ptr, (size_t)size);
    pool->release_now(chunk);
  });
}

Buffer* copy_buffer(Buffer* src, Device* d) {
  if (src->deleted) fail(PJRT_Error_Code_FAILED_PRECONDITION, "copy of a deleted buffer");
  if (d != src->device) unimplemented("copies between devices are not supported");
  Client* c = src->client;
  auto b = std::make_unique<Buffer>();
  b->client = c;
  b->device = d;
  b->dtype = src->dtype;
  b->dims = src->dims;
  b->minor_to_major = src->minor_to_major;
  Status err(PJRT_Error_Code_OK, "");
  if (buffer_error(src, &err)) {  // the copy of an error buffer is an error buffer
    b->ready = error_event(err);
    return b.release();
  }
  b->mem = c->allocate(d, src->bytes());
  std::lock_guard<std::recursive_mutex> lk(d->launch_mu);
  HIP_CHECK(hipSetDevice(d->hip_ordinal));
  if (src->bytes()) HIP_CHECK(hipMemcpyAsync(b->mem->ptr, src->mem->ptr, src->bytes(), hipMemcpyDeviceToDevice, d->stream));
  b->ready = c->record_event(d);
  return b.release();
}

// ------------------------------------------------------------------------------------------------ compile
static std::string fnv_hex(const std::string& a, const std::string& b) {
  uint64_t h = 1469598103934665603ull;
  for (unsigned char ch : a) { h ^= ch; h *= 1099511628211ull; }
  for (unsigned char ch : b) { h ^= ch; h *= 1099511628211ull; }
  char buf[32];
  snprintf(buf, sizeof(buf), "%016llx", (unsigned long long)h);
  return buf;
}

std::shared_ptr<Executable> compile_program(Client* c, const std::string& code, const std::string& format,
                                            const std::string& options) {
  if (format != "mlir") unimplemented("program format '" + format + "' is not supported; pass StableHLO as \"mlir\"");
  struct CompileSpan {  // the compilation's host span, for started profiler sessions
    int64_t begin = wall_clock_ns();
    ~CompileSpan() {
      try {
        if (profiler_sessions_active()) profiler_record_host("compile main", begin, wall_clock_ns());
      } catch (...) {
      }
    }
  } span;
  auto exe = std::make_shared<Executable>();
  exe->options = decode_compile_options(options);
  exe->device_index = choose_device(exe->options, c->device_ptrs.size());
  Graph g = is_mlir_bytecode(code.data(), code.size()) ? parse_mlir_bytecode(code, "main") : parse_mlir_text(code, "main");
  PlanOptions po;
  po.fast_paths = c->fast_paths;
  exe->plan = build_plan(g, po);
  exe->name = "main";
  exe->fingerprint = fnv_hex(code, options);
  exe->program_text = code;
  exe->compile_options = options;
  for (auto& t : exe->plan.output_types) {
    exe->output_types.push_back((PJRT_Buffer_Type)t.dtype);
    exe->output_ranks.push_back(t.shape.size());
    for (auto d : t.shape) exe->output_dims_flat.push_back(d);
    static const char* kDevice = "device";
    exe->output_memory_kinds.push_back(kDevice);
    exe->output_memory_kind_sizes.push_back(6);
  }
  auto row_major_layout = [](size_t rank) {
    auto l = std::make_unique<MemoryLayout>();
    for (size_t i = 0; i < rank; ++i) l->minor_to_major.push_back((int64_t)(rank - 1 - i));
    return l;
  };
  for (auto& t : exe->plan.param_types) {
    exe->param_layouts.push_back(row_major_layout(t.shape.size()));
    exe->param_layout_ptrs.push_back(exe->param_layouts.back().get());
  }
  for (auto& t : exe->plan.output_types) {
    exe->output_layouts.push_back(row_major_layout(t.shape.size()));
    exe->output_layout_ptrs.push_back(exe->output_layouts.back().get());
  }
  for (size_t i = 0; i < exe->plan.param_types.size(); ++i) {
    static const char* kDevice = "device";
    exe->param_memory_kinds.push_back(kDevice);
    exe->param_memory_kind_sizes.push_back(6);
  }
  static const char* kFlops = "flops";
  static const char* kBytes = "bytes accessed";
  PJRT_NamedValue f{};
  f.struct_size = sizeof(PJRT_NamedValue);
  f.name = kFlops;
  f.name_size = 5;
  f.type = PJRT_NamedValue_kFloat;
  f.float_value = (float)exe->plan.total_flops;
  f.value_size = 1;
  PJRT_NamedValue by = f;
  by.name = kBytes;
  by.name_size = strlen(kBytes);
  by.float_value = (float)exe->plan.total_bytes;
  exe->cost_properties = {f, by};
  // upload non-splat constants once, to the executable's device
  exe->constants.resize(exe->plan.slots.size());
  if (c->device_ptrs.empty()) return exe;  // compile-only client
  Device* d = c->device_ptrs.at(exe->device_index);
  for (size_t s = 0; s < exe->plan.slots.size(); ++s) {
    const Slot& sl = exe->plan.slots[s];
    if (sl.kind != Slot::CONSTANT) continue;
    auto m = c->allocate(d, sl.literal.size());
    std::lock_guard<std::recursive_mutex> lk(d->launch_mu);
    HIP_CHECK(hipSetDevice(d->hip_ordinal));
    if (!sl.literal.empty()) {
      HIP_CHECK(hipMemcpyAsync(m->ptr, sl.literal.data(), sl.literal.size(), hipMemcpyHostToDevice, d->stream));
      HIP_CHECK(hipStreamSynchronize(d->stream));
    }
    exe->constants[s] = m;
  }
  return exe;
}

// Serialized executable: "RYFTEXE1", then the program bytes and the compile-options bytes, each after its u64
// length. Deserialisation compiles the program again (plans are cheap to rebuild; the kernels live in the plugin).
static const char kExeMagic[8] = {'R', 'Y', 'F', 'T', 'E', 'X', 'E', '1'};

std::string serialize_executable(const Executable& e) {
  std::string out(kExeMagic, sizeof(kExeMagic));
  auto put = [&](const std::string& v) {
    uint64_t n = v.size();
    out.append((const char*)&n, sizeof(n));
    out.append(v);
  };
  put(e.program_text);
  put(e.compile_options);
  return out;
}

std::shared_ptr<Executable> deserialize_executable(Client* c, const char* data, size_t size, const std::string* options) {
  if (!data || size < sizeof(kExeMagic) || memcmp(data, kExeMagic, sizeof(kExeMagic)) != 0)
    invalid("not a serialized executable of this plugin (bad header)");
  size_t pos = sizeof(kExeMagic);
  auto get = [&](const char* what) {
    uint64_t n = 0;
    if (size - pos < sizeof(n)) invalid(std::string("serialized executable is truncated (") + what + " length)");
    memcpy(&n, data + pos, sizeof(n));
    pos += sizeof(n);
    if (n > size - pos) invalid(std::string("serialized executable is truncated (") + what + ")");
    std::string v(data + pos, (size_t)n);
    pos += (size_t)n;
    return v;
  };
  std::string code = get("program");
  std::string opts = get("compile options");
  if (pos != size) invalid("serialized executable has trailing bytes");
  return compile_program(c, code, "mlir", options ? *options : opts);
}

// ------------------------------------------------------------------------------------------------ execute
TimingEvents::TimingEvents() {
  HIP_CHECK(hipEventCreate(&start));
  HIP_CHECK(hipEventCreate(&stop));
}
TimingEvents::~TimingEvents() {
  if (start) (void)hipEventDestroy(start);
  if (stop) (void)hipEventDestroy(stop);
}

bool enqueue_steps(Client* c, const Plan& plan, void* const* ptr, hipStream_t st, hipEvent_t done, bool prof,
                   int device_id, bool profilable) {
  const bool record = profilable && profiler_sessions_active();  // started profiler sessions take the events too
  const bool timed = prof || record;
  constexpr size_t kBlock = std::max({sizeof(EwProgram), sizeof(ReduceArgs), sizeof(GemmArgs), sizeof(RowArgs),
                                      sizeof(AttnArgs), sizeof(WindowArgs), sizeof(GatherArgs),
                                      sizeof(ReduceBodyArgs), sizeof(ScatterArgs)});
  alignas(64) static thread_local unsigned char block[kBlock + 64];
  bool recorded = false;
  for (size_t si = 0; si < plan.steps.size(); ++si) {
    const Step& step = plan.steps[si];
    hipEvent_t carry = (!timed && si + 1 == plan.steps.size() && step.kind != Step::COPY) ? done : nullptr;
    recorded |= carry != nullptr;
    StepTiming tm;
    if (timed) {
      tm.name = step.name;
      tm.flops = step.flops;
      tm.bytes = step.bytes;
      tm.device = device_id;
      tm.host_ns = wall_clock_ns();
      tm.ev = std::make_shared<TimingEvents>();
      // kernel steps: the first launch records the start, the last the stop (the kernels' own duration)
      if (step.kind == Step::COPY) HIP_CHECK(hipEventRecord(tm.ev->start, st));
      else pending_start() = tm.ev->start;
    }
    if (step.kind == Step::COPY) {
      void* src = (char*)ptr[step.patches[0].second] + step.copy.src_offset;
      void* dst = ptr[step.patches[1].second];
      if (step.copy.bytes && dst != src)  // (a result computed in place over its donated parameter: nothing to copy)
        HIP_CHECK(hipMemcpyAsync(dst, src, (size_t)step.copy.bytes, hipMemcpyDeviceToDevice, st));
    } else {
      size_t sz = step.kind == Step::ELEMENTWISE ? sizeof(EwProgram)
                  : step.kind == Step::REDUCE    ? sizeof(ReduceArgs)
                  : step.kind == Step::GEMM      ? sizeof(GemmArgs)
                  : step.kind == Step::ROW       ? sizeof(RowArgs)
                  : step.kind == Step::WINDOW    ? sizeof(WindowArgs)
                  : step.kind == Step::GATHER    ? sizeof(GatherArgs)
                  : step.kind == Step::SCATTER   ? sizeof(ScatterArgs)
                  : step.kind == Step::REDUCE_BODY ? sizeof(ReduceBodyArgs)
                                                 : sizeof(AttnArgs);
      memcpy(block, const_cast<Step&>(step).args_block(), sz);
      for (auto& p : step.patches) {
        void** f = (void**)(block + p.first);
        *f = (char*)ptr[p.second] + (uintptr_t)(*f);
      }
      hipEvent_t last = timed ? tm.ev->stop : carry;
      switch (step.kind) {
        case Step::ELEMENTWISE: launch_elementwise(*(EwProgram*)block, st, last); break;
        case Step::REDUCE: launch_reduce(*(ReduceArgs*)block, st, last); break;
        case Step::ROW: launch_row(*(RowArgs*)block, st, last); break;
        case Step::GEMM: launch_gemm(*(GemmArgs*)block, st, last); break;
        case Step::ATTENTION: launch_attention(*(AttnArgs*)block, st, last); break;
        case Step::WINDOW: launch_window(*(WindowArgs*)block, st, last); break;
        case Step::GATHER: launch_gather(*(GatherArgs*)block, st, last); break;
        case Step::SCATTER: launch_scatter(*(ScatterArgs*)block, st, last); break;
        case Step::REDUCE_BODY: launch_reduce_body(*(ReduceBodyArgs*)block, st, last); break;
        default: recorded = false; break;
      }
      if (hipEvent_t unused = pending_start()) {  // no launch took it
        pending_start() = nullptr;
        HIP_CHECK(hipEventRecord(unused, st));
      }
    }
    if (timed) {
      if (step.kind == Step::COPY) HIP_CHECK(hipEventRecord(tm.ev->stop, st));
      if (record) profiler_record_step(tm);
      if (prof) {
        std::lock_guard<std::mutex> pl(c->prof_mu);
        c->timings.push_back(tm);
      }
    }
  }
  return recorded;
}

EventPtr execute(LoadedExecutable* le, Device* d, Buffer* const* args, size_t num_args, std::vector<Buffer*>* outputs,
                 const int64_t* non_donatable, size_t num_non_donatable, int launch_id) {
  const int64_t host_begin = wall_clock_ns();
  Executable& exe = *le->exe;
  const Plan& plan = exe.plan;
  Client* c = le->client;
  if (!d) fail(PJRT_Error_Code_FAILED_PRECONDITION, "this client was created compile-only and cannot execute");
  if (num_args != plan.param_slots.size())
    invalid("executable expects " + std::to_string(plan.param_slots.size()) + " argument(s) but got " + std::to_string(num_args));
  for (size_t i = 0; i < num_args; ++i) {
    Buffer* b = args[i];
    if (!b) invalid("argument " + std::to_string(i) + " is null");
    if (b->deleted) fail(PJRT_Error_Code_FAILED_PRECONDITION, "argument " + std::to_string(i) + " has been deleted");
    const TensorType& t = plan.param_types[i];
    if (b->dtype != t.dtype || b->dims != t.shape)
      invalid("argument " + std::to_string(i) + " has type " + TensorType{b->dtype, b->dims}.str() + " but the program expects " + t.str());
    if (b->device != d) invalid("argument " + std::to_string(i) + " lives on another device");
  }
  // an error buffer among the arguments fails the execution with its error
  for (size_t i = 0; i < num_args; ++i) {
    Status err(PJRT_Error_Code_OK, "");
    if (buffer_error(args[i], &err)) throw err;
  }
  // donation (XLA's aliasing semantics): an argument aliased to a result is donated unless the caller marked it
  // non-donatable, in which case the result simply gets a buffer of its own
  std::vector<int> donated_to(num_args, -1);  // argument → result
  for (size_t o = 0; o < plan.output_alias.size(); ++o) {
    const int p = plan.output_alias[o];
    if (p < 0) continue;
    bool keep = false;
    for (size_t k = 0; k < num_non_donatable; ++k) {
      if (non_donatable[k] < 0 || (size_t)non_donatable[k] >= num_args)
        invalid("non-donatable input index " + std::to_string(non_donatable[k]) + " is out of range");
      keep |= non_donatable[k] == p;
    }
    if (keep) continue;
    Buffer* b = args[p];
    if (b->external_refs.load() > 0)
      invalid("argument " + std::to_string(p) + " is donated but has external references");
    for (size_t i = 0; i < num_args; ++i)
      if (i != (size_t)p && args[i] == b)
        invalid("argument " + std::to_string(p) + " is donated but the same buffer is also argument " + std::to_string(i));
    donated_to[p] = (int)o;
  }
  std::vector<void*> ptr(plan.slots.size(), nullptr);
  std::vector<std::shared_ptr<DeviceMem>> hold(plan.slots.size());
  for (size_t s = 0; s < plan.slots.size(); ++s) {
    const Slot& sl = plan.slots[s];
    switch (sl.kind) {
      case Slot::PARAM: ptr[s] = args[sl.index]->mem->ptr; break;
      case Slot::CONSTANT: ptr[s] = exe.constants[s]->ptr; break;
      case Slot::OUTPUT: {
        const int p = plan.output_alias.empty() ? -1 : plan.output_alias[sl.index];
        if (p >= 0 && donated_to[p] == sl.index && plan.output_in_place[sl.index]) {
          hold[s] = args[p]->mem;  // computed straight into the donated buffer
          ptr[s] = hold[s]->ptr;
          break;
        }
        hold[s] = c->allocate(d, sl.type.bytes());
        ptr[s] = hold[s]->ptr;
        break;
      }
      case Slot::TEMP:
        hold[s] = c->allocate(d, sl.type.bytes());
        ptr[s] = hold[s]->ptr;
        break;
    }
  }
  EventPtr done;
  {
    std::lock_guard<std::recursive_mutex> lk(d->launch_mu);
    HIP_CHECK(hipSetDevice(d->hip_ordinal));
    hipStream_t st = d->stream;
    bool prof;
    {
      std::lock_guard<std::mutex> pl(c->prof_mu);
      prof = c->profiling;
    }
    // The execution's completion event rides on its last kernel launch when it can (no separate marker packet
    // between consecutive executions); otherwise it is recorded after the last step.
    done = std::make_shared<EventState>();
    HIP_CHECK(hipEventCreateWithFlags(&done->hip_event, hipEventDisableTiming));
    const bool recorded = enqueue_steps(c, plan, ptr.data(), st, done->hip_event, prof, d->id);
    if (!recorded) HIP_CHECK(hipEventRecord(done->hip_event, st));
    // Nothing runs on this event's completion unless a callback is registered, so it is not queued on the
    // completion worker.
    done->lazy_owner = c;
  }
  {
    // in-flight record for poison_execution: entries whose event is gone or ready are dropped from the front; the
    // oldest beyond kMaxInflight are dropped too (on one in-order stream they have long finished)
    constexpr size_t kMaxInflight = 1024;
    std::lock_guard<std::mutex> lk(d->inflight_mu);
    while (!d->inflight.empty()) {
      EventPtr e = d->inflight.front().second.lock();
      bool gone = !e;
      if (e) {
        std::lock_guard<std::mutex> el(e->mu);
        gone = e->ready;
      }
      if (!gone && d->inflight.size() < kMaxInflight) break;
      d->inflight.pop_front();
    }
    d->inflight.emplace_back(launch_id, done);
  }
  outputs->clear();
  for (size_t i = 0; i < plan.output_slots.size(); ++i) {
    int s = plan.output_slots[i];
    auto b = std::make_unique<Buffer>();
    b->client = c;
    b->device = d;
    b->dtype = plan.slots[s].type.dtype;
    b->dims = plan.slots[s].type.shape;
    for (int k = (int)b->dims.size() - 1; k >= 0; --k) b->minor_to_major.push_back(k);
    b->mem = hold[s];
    b->ready = done;
    outputs->push_back(b.release());
  }
  // donated arguments are gone; their memory lives on in the result that took it over, or returns to the allocator
  // (ordered after this execution's reads on the device's one stream)
  for (size_t i = 0; i < num_args; ++i)
    if (donated_to[i] >= 0) {
      args[i]->deleted = true;
      args[i]->mem.reset();
    }
  if (profiler_sessions_active()) profiler_record_host("execute " + exe.name, host_begin, wall_clock_ns());
  return done;
}

bool poison_execution(Device* d, int launch_id, const Status& err) {
  std::vector<EventPtr> cand;
  {
    std::lock_guard<std::mutex> lk(d->inflight_mu);
    for (auto& e : d->inflight)
      if (e.first == launch_id)
        if (EventPtr p = e.second.lock()) cand.push_back(std::move(p));
  }
  // oldest first; poll() resolves executions whose device work has ended (without the device lock held: it may run
  // OnReady callbacks)
  for (EventPtr& e : cand) {
    if (e->poll()) continue;
    if (e->poison(err)) return true;
  }
  return false;
}

std::string kernel_timing_json(Client* c) {
  for (auto& d : c->devices) {
    (void)hipSetDevice(d->hip_ordinal);
    HIP_CHECK(hipStreamSynchronize(d->stream));
  }
  struct Agg {
    int64_t count = 0;
    double ms = 0, min_ms = 1e30, max_ms = 0, flops = 0, bytes = 0;
    std::vector<double> samples;
  };
  std::map<std::string, Agg> agg;
  std::vector<std::string> order;
  {
    std::lock_guard<std::mutex> lk(c->prof_mu);
    for (auto& t : c->timings) {
      float ms = 0;
      HIP_CHECK(hipEventElapsedTime(&ms, t.ev->start, t.ev->stop));
      if (!agg.count(t.name)) order.push_back(t.name);
      Agg& a = agg[t.name];
      a.count++;
      a.ms += ms;
      a.min_ms = std::min(a.min_ms, (double)ms);
      a.max_ms = std::max(a.max_ms, (double)ms);
      a.samples.push_back(ms);
      a.flops += t.flops;
      a.bytes += t.bytes;
    }
    c->timings.clear();
  }
  std::ostringstream os;
  os << "{";
  bool first = true;
  for (auto& n : order) {
    Agg& a = agg[n];
    std::sort(a.samples.begin(), a.samples.end());
    const size_t h = a.samples.size() / 2;
    const double median = a.samples.size() % 2 ? a.samples[h] : 0.5 * (a.samples[h - 1] + a.samples[h]);
    os << (first ? "" : ",") << "\"" << n << "\":{\"count\":" << a.count << ",\"total_ms\":" << a.ms
       << ",\"median_us\":" << 1e3 * median
       << ",\"avg_us\":" << 1e3 * a.ms / a.count << ",\"min_us\":" << 1e3 * a.min_ms << ",\"max_us\":" << 1e3 * a.max_ms
       << ",\"flops\":" << a.flops / a.count << ",\"bytes\":" << a.bytes / a.count << "}";
    first = false;
  }
  os << "}";
  return os.str();
}

}  // namespace ryft
