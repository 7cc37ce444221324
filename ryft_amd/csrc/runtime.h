// Runtime objects behind the PJRT handles: one client per process-visible MI355X, one HIP stream per device,
// a caching device allocator, pinned staging for host transfers, and events completed by a worker thread.
#pragma once

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <condition_variable>
#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "common.h"
#include "planner.h"

namespace ryft {

#define HIP_CHECK(expr)                                                                                    \
  do {                                                                                                     \
    hipError_t _e = (expr);                                                                                \
    if (_e != hipSuccess)                                                                                  \
      ::ryft::fail(PJRT_Error_Code_INTERNAL, std::string(#expr) + " failed: " + hipGetErrorString(_e));    \
  } while (0)

struct Client;

// A PJRT_Error object (pjrt_api.cc); the caller owns it.
PJRT_Error* make_pjrt_error(PJRT_Error_Code code, const std::string& msg, const Payload& payload = {});

// ------------------------------------------------------------------------------------------------ events
struct EventState {
  std::mutex mu;
  std::condition_variable cv;
  bool ready = false;
  PJRT_Error_Code code = PJRT_Error_Code_OK;
  std::string message;
  Payload payload;
  // Set by PJRT_Device_PoisonExecution before the event is ready: it then turns ready with this error (code,
  // message and payload above) whatever the device work's own outcome.
  bool poisoned = false;
  std::vector<std::pair<PJRT_Event_OnReadyCallback, void*>> callbacks;
  hipEvent_t hip_event = nullptr;  // completion marker on the device stream (null for host events)
  std::function<void()> on_complete;  // host work run before the event turns ready (e.g. staging → user copy)
  // Execution completion events are resolved on demand (await, query) rather than by the client's completion
  // worker; the first OnReady callback registered before completion hands the event to `lazy_owner`'s worker.
  struct Client* lazy_owner = nullptr;
  bool queued = false;

  ~EventState();
  // Marks the event ready (idempotent) and runs the registered callbacks on this thread.
  void set_ready(PJRT_Error_Code c, const std::string& msg);
  // Blocks until the event is ready; synchronizes its HIP event on the calling thread when it has one.
  void wait();
  bool poll();
  // The error this event already carries — set, or poisoned and pending — if any (buffers defined by it are then
  // error buffers: their consumers fail with it instead of reading their memory).
  bool error_now(Status* out);
  // Poisons a pending event with `err`; false if the event is already ready.
  bool poison(const Status& err);
};
using EventPtr = std::shared_ptr<EventState>;
// An event that is ready with `err` from the start.
EventPtr error_event(const Status& err);

struct Event {  // PJRT_Event
  EventPtr state;
};

// ------------------------------------------------------------------------------------------------ memory
class DeviceAllocator {
 public:
  explicit DeviceAllocator(int device) : device_(device) {}
  ~DeviceAllocator();
  void* allocate(size_t bytes);
  void release(void* p);
  int64_t bytes_in_use() const { return in_use_; }
  int64_t peak_bytes() const { return peak_; }
  int64_t num_allocs() const { return allocs_; }

 private:
  static size_t round_size(size_t bytes);
  void trim();
  int device_;
  std::mutex mu_;
  std::map<size_t, std::vector<void*>> free_;  // size class → cached blocks
  std::map<void*, size_t> live_;
  int64_t in_use_ = 0, peak_ = 0, allocs_ = 0;
};

struct DeviceMem {
  void* ptr = nullptr;
  size_t bytes = 0;
  DeviceAllocator* alloc = nullptr;
  ~DeviceMem() {
    if (ptr && alloc) alloc->release(ptr);
  }
};

class PinnedPool {
 public:
  ~PinnedPool();
  struct Chunk {
    void* ptr = nullptr;
    size_t bytes = 0;
    hipEvent_t last_use = nullptr;
    bool busy = false;
  };
  Chunk* acquire(size_t bytes);
  void release(Chunk* c, hipStream_t stream);  // reusable once the stream passes this point
  void release_now(Chunk* c);

 private:
  std::mutex mu_;
  std::vector<std::unique_ptr<Chunk>> chunks_;
};

// ------------------------------------------------------------------------------------------------ devices
struct Memory;
struct Device {  // PJRT_Device and PJRT_DeviceDescription
  Client* client = nullptr;
  int id = 0;
  int hip_ordinal = 0;
  std::string kind, debug, to_string, arch;
  std::vector<PJRT_NamedValue> attributes;
  std::vector<std::string> attribute_strings;
  std::vector<Memory*> memories;
  Memory* default_memory = nullptr;
  hipStream_t stream = nullptr;
  std::unique_ptr<DeviceAllocator> allocator;
  std::recursive_mutex launch_mu;  // serializes enqueue on the device stream
  // Executions enqueued on this device and not yet seen finished, oldest first, by launch id
  // (PJRT_ExecuteOptions.launch_id), for PJRT_Device_PoisonExecution.
  std::mutex inflight_mu;
  std::deque<std::pair<int, std::weak_ptr<EventState>>> inflight;
};

struct Memory {  // PJRT_Memory
  Client* client = nullptr;
  int id = 0;
  std::string kind = "device";
  std::string debug, to_string;
  std::vector<Device*> devices;
};

// ------------------------------------------------------------------------------------------------ buffers
struct Buffer {  // PJRT_Buffer
  Client* client = nullptr;
  Device* device = nullptr;
  DType dtype = DType::INVALID;
  std::vector<int64_t> dims;
  std::shared_ptr<DeviceMem> mem;
  EventPtr ready;
  std::atomic<bool> deleted{false};
  std::atomic<int> external_refs{0};
  std::vector<int64_t> minor_to_major;
  size_t bytes() const { return (size_t)num_elements(dims) * dtype_size(dtype); }
};

// ------------------------------------------------------------------------------------------------ executables
struct MemoryLayout {  // PJRT_Layouts_MemoryLayout: dense, untiled
  std::vector<int64_t> minor_to_major;
};

// The CompileOptionsProto fields the plugin acts on (crates/ryft-xla-sys/src/protos.rs:3298-3346, 2391-2530).
struct CompileOptions {
  int64_t device_ordinal = -1;  // -1: the client's first device
  int64_t replica_count = 1, partition_count = 1;
  bool use_spmd_partitioning = false;
  bool tupled_arguments = false;
  bool portable = false;
  int precision = 0;  // matrix_unit_operand_precision: 0 default, 1 high, 2 highest (f32 dots run f32 MFMAs always)
  int64_t assignment_replicas = 0, assignment_computations = 0;
  std::vector<int64_t> assignment_ids;  // device ids of an explicit device assignment (empty: none)
};
// Decodes serialized compile options (empty bytes: the defaults). Malformed bytes are INVALID_ARGUMENT; more than one
// replica or partition, tupled parameters or a multi-device assignment are UNIMPLEMENTED.
CompileOptions decode_compile_options(const std::string& bytes);
// Index of the client device an executable with these options runs on (num_devices 0: compile-only, unchecked).
int choose_device(const CompileOptions& o, size_t num_devices);

struct Executable {  // PJRT_Executable (shared by the loaded executable and every view handed out)
  std::string name;
  std::string fingerprint;
  std::string program_text;
  std::string compile_options;
  CompileOptions options;
  int device_index = 0;  // the client device it was compiled for (constants live there)
  Plan plan;
  std::vector<PJRT_Buffer_Type> output_types;
  std::vector<int64_t> output_dims_flat;
  std::vector<size_t> output_ranks;
  std::vector<const char*> output_memory_kinds;
  std::vector<size_t> output_memory_kind_sizes;
  std::vector<const char*> param_memory_kinds;
  std::vector<size_t> param_memory_kind_sizes;
  // row-major layouts of the parameters and results, owned here (the layouts extension lends them out)
  std::vector<std::unique_ptr<MemoryLayout>> param_layouts, output_layouts;
  std::vector<MemoryLayout*> param_layout_ptrs, output_layout_ptrs;
  std::vector<PJRT_NamedValue> cost_properties;
  std::vector<std::shared_ptr<DeviceMem>> constants;  // by slot (null for non-constant slots)
};

struct ExecuteContext {};  // PJRT_ExecuteContext: carries nothing the plugin reads

struct ExecutableView {  // what PJRT_Executable* points to
  std::shared_ptr<Executable> exe;
};

struct LoadedExecutable {  // PJRT_LoadedExecutable
  Client* client = nullptr;
  std::shared_ptr<Executable> exe;
  std::vector<Device*> devices;
  std::vector<PJRT_LogicalDeviceIds> logical_ids;
  std::atomic<bool> deleted{false};
};

// ------------------------------------------------------------------------------------------------ client
// HIP events recorded by a plan step's first and last kernel launch (destroyed with the last holder).
struct TimingEvents {
  hipEvent_t start = nullptr, stop = nullptr;
  TimingEvents();
  ~TimingEvents();
  TimingEvents(const TimingEvents&) = delete;
  TimingEvents& operator=(const TimingEvents&) = delete;
};

struct StepTiming {
  std::string name;
  double flops = 0, bytes = 0;
  int device = 0;        // PJRT device id
  int64_t host_ns = 0;   // wall clock when the step was enqueued
  std::shared_ptr<TimingEvents> ev;
};

// ------------------------------------------------------------------------------------------------ profiler
// Sessions of the PJRT profiler extension (profiler.cc). While at least one is started, executions record their
// steps' HIP events (and their own host spans) into every started session.
bool profiler_sessions_active();
void profiler_record_step(const StepTiming& t);
void profiler_record_host(const std::string& name, int64_t begin_ns, int64_t end_ns);
int64_t wall_clock_ns();
extern PJRT_Profiler_Extension g_profiler_extension;  // the extension's table (chained into the PJRT_Api)

struct Client {  // PJRT_Client
  std::string platform_name = "rocm";
  std::string platform_version;
  std::vector<std::unique_ptr<Device>> devices;
  std::vector<Device*> device_ptrs;
  std::vector<std::unique_ptr<Memory>> memories;
  std::vector<Memory*> memory_ptrs;
  PinnedPool pinned;
  bool fast_paths = true;  // planner option (PlanOptions::fast_paths)

  // completion worker: fires OnReady callbacks / host-side copy completions in stream order
  std::mutex q_mu;
  std::condition_variable q_cv;
  std::deque<EventPtr> queue;
  bool stopping = false;
  std::thread worker;

  // kernel timing (profiling extension)
  std::mutex prof_mu;
  bool profiling = false;
  std::vector<StepTiming> timings;

  Client(const std::vector<int>& visible, bool compile_only);
  // Drains the completion worker (it exits once its queue is empty) and the device streams. Called by the
  // destructor, and at process exit for clients the host never destroyed.
  void stop_worker();
  ~Client();
  void enqueue_completion(const EventPtr& e);
  EventPtr record_event(Device* d, std::function<void()> on_complete = nullptr);
  std::shared_ptr<DeviceMem> allocate(Device* d, size_t bytes);
};

// Creates a device buffer holding a copy of `data` (dense row-major unless byte_strides is given).
Buffer* buffer_from_host(Client* c, Device* d, const void* data, DType t, const std::vector<int64_t>& dims,
                         const int64_t* byte_strides, size_t num_byte_strides, EventPtr* done_with_host);
// Starts a device → host copy into `dst`; returns the completion event.
EventPtr buffer_to_host(Buffer* b, void* dst, size_t dst_size);
// Compiles a StableHLO program.
// Executable bytes for PJRT_Executable_Serialize, and the executable they describe (compiled again on this client;
// `options`, when given, replaces the serialized compile options).
std::string serialize_executable(const Executable& e);
std::shared_ptr<Executable> deserialize_executable(Client* c, const char* data, size_t size, const std::string* options);
// A byte range of a buffer's device bytes → host memory; the event completes when `dst` holds the bytes.
EventPtr buffer_raw_to_host(Buffer* b, void* dst, int64_t offset, int64_t size);
std::shared_ptr<Executable> compile_program(Client* c, const std::string& code, const std::string& format,
                                            const std::string& options);
// Enqueues one execution; fills outputs and returns the completion event. Arguments that the program aliases to a
// result are donated unless their index is in `non_donatable`: the result takes over (or replaces) the argument's
// device memory and the argument buffer is marked deleted. An argument that is an error buffer (made by
// PJRT_Client_CreateErrorBuffer, or a result of a poisoned execution) fails the call with its error, before anything
// is enqueued. The execution is recorded under `launch_id` for poison_execution.
EventPtr execute(LoadedExecutable* le, Device* d, Buffer* const* args, size_t num_args, std::vector<Buffer*>* outputs,
                 const int64_t* non_donatable = nullptr, size_t num_non_donatable = 0, int launch_id = 0);
// PJRT_Device_PoisonExecution: the earliest execution on `d` under `launch_id` that has not finished turns ready
// with `err` when its device work ends (its results become error buffers at once); false when every such execution
// has finished already. The device work itself runs to its end.
bool poison_execution(Device* d, int launch_id, const Status& err);
// Enqueues every step of `plan` on `st`, slot s living at ptr[s] (the caller has made the plan's device current).
// `done` (optional) is recorded by the last kernel launch when it can; returns whether it was. With `prof`, each
// step's first and last launch record timing events appended to c->timings; while a profiler session is started,
// they are recorded for it too (device_id names the device in its trace) unless `profilable` is false. Allocates no
// device memory; creates no HIP object unless timing.
bool enqueue_steps(Client* c, const Plan& plan, void* const* ptr, hipStream_t st, hipEvent_t done, bool prof,
                   int device_id = 0, bool profilable = true);
// Device address of the allocation-free entry point's scratch array on a GPU (looked up once per device, with
// that device current; null if the lookup fails), and its size.
void* noalloc_scratch(int hip_ordinal);
size_t noalloc_scratch_bytes();
// Copies a buffer to another buffer on the same device.
Buffer* copy_buffer(Buffer* src, Device* d);

std::string kernel_timing_json(Client* c);

}  // namespace ryft
