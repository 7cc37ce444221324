// Allocation-free execution of a loaded executable: RyftMi355x_ExecuteNoAlloc (include/ryft_mi355x.h).
//
// The caller brings the device memory of the parameters and results; the plan's intermediates (TEMP slots: split-K
// partial sums, a normalised activation between two launches, ...) live in `scratch`, a file-scope device array of
// kScratchBytes that each GPU holds from the library's load until the process ends. Nothing here calls hipMalloc,
// hipFree or any other allocating routine, so the entry point serves callers that cannot allocate (code under HIP
// graph capture, tight serving loops).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "../runtime.h"
#include "ryft_mi355x.h"

namespace ryft {
namespace {

constexpr size_t kScratchBytes = (size_t)64 << 20;  // 64 MiB per GPU
constexpr int kMaxDevices = 64;
constexpr size_t kMaxSlots = 1024;

// Every call on a GPU shares that GPU's copy. No kernel reads an intermediate before writing it, so nothing needs
// clearing between calls; calls that overlap on one GPU (two streams, or two host threads) race on it.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Device address of each GPU's copy (the host-side name `scratch` is not one: kernels get these pointers).
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

thread_local char g_message[256];

int report(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int report(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_message, sizeof(g_message), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace

void* noalloc_scratch(int hip_ordinal) {
  if (hip_ordinal < 0 || hip_ordinal >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[hip_ordinal]) {
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) return nullptr;
    if (hipSetDevice(hip_ordinal) != hipSuccess) return nullptr;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    (void)hipSetDevice(prev);
    if (e != hipSuccess || !p) return nullptr;
    g_scratch_ptr[hip_ordinal] = p;
  }
  return g_scratch_ptr[hip_ordinal];
}

size_t noalloc_scratch_bytes() { return kScratchBytes; }

}  // namespace ryft

using namespace ryft;

extern "C" int RyftMi355x_ExecuteNoAlloc(PJRT_LoadedExecutable* executable, const void* const* inputs,
                                         const size_t* input_sizes, size_t num_inputs, void* const* outputs,
                                         const size_t* output_sizes, size_t num_outputs, void* stream,
                                         const char** error_message) {
  g_message[0] = 0;
  if (error_message) *error_message = g_message;
  if (!executable) return report(PJRT_Error_Code_INVALID_ARGUMENT, "executable is null");
  auto* le = reinterpret_cast<LoadedExecutable*>(executable);
  if (le->deleted) return report(PJRT_Error_Code_FAILED_PRECONDITION, "executable has been deleted");
  if (le->devices.empty() || !le->devices[0])
    return report(PJRT_Error_Code_FAILED_PRECONDITION, "executable was compiled without a device (compile-only client)");
  Device* d = le->devices[0];
  const Executable& exe = *le->exe;
  const Plan& plan = exe.plan;
  if (num_inputs != plan.param_slots.size())
    return report(PJRT_Error_Code_INVALID_ARGUMENT, "executable expects %zu input(s) but got %zu",
                  plan.param_slots.size(), num_inputs);
  if (num_outputs != plan.output_slots.size())
    return report(PJRT_Error_Code_INVALID_ARGUMENT, "executable has %zu output(s) but got %zu",
                  plan.output_slots.size(), num_outputs);
  if (plan.slots.size() > kMaxSlots)
    return report(PJRT_Error_Code_UNIMPLEMENTED, "plan has %zu buffer slots (at most %zu)", plan.slots.size(), kMaxSlots);
  if ((num_inputs && (!inputs || !input_sizes)) || (num_outputs && (!outputs || !output_sizes)))
    return report(PJRT_Error_Code_INVALID_ARGUMENT, "input / output pointer or size array is null");

  // Intermediates, each at a 256-byte aligned offset of the scratch array (the alignment the planner assumes of
  // every slot's base).
  size_t need = 0;
  for (const Slot& sl : plan.slots)
    if (sl.kind == Slot::TEMP) need += (sl.type.bytes() + 255) & ~(size_t)255;
  if (need > kScratchBytes)
    return report(PJRT_Error_Code_RESOURCE_EXHAUSTED,
                  "executable needs %zu bytes of intermediates; the allocation-free scratch holds %zu", need,
                  kScratchBytes);

  void* ptr[kMaxSlots];
  char* base = nullptr;
  if (need) {
    base = (char*)noalloc_scratch(d->hip_ordinal);
    if (!base) return report(PJRT_Error_Code_INTERNAL, "scratch address of device %d unavailable", d->hip_ordinal);
  }
  size_t off = 0;
  for (size_t s = 0; s < plan.slots.size(); ++s) {
    const Slot& sl = plan.slots[s];
    const size_t bytes = sl.type.bytes();
    switch (sl.kind) {
      case Slot::PARAM: {
        const void* p = inputs[sl.index];
        if (input_sizes[sl.index] != bytes)
          return report(PJRT_Error_Code_INVALID_ARGUMENT, "input %d holds %zu bytes; the program expects %zu",
                        sl.index, input_sizes[sl.index], bytes);
        if (bytes && (!p || ((uintptr_t)p & 255)))
          return report(PJRT_Error_Code_INVALID_ARGUMENT, "input %d must be a non-null 256-byte aligned device pointer",
                        sl.index);
        ptr[s] = const_cast<void*>(p);
        break;
      }
      case Slot::OUTPUT: {
        void* p = outputs[sl.index];
        if (output_sizes[sl.index] != bytes)
          return report(PJRT_Error_Code_INVALID_ARGUMENT, "output %d holds %zu bytes; the program writes %zu",
                        sl.index, output_sizes[sl.index], bytes);
        if (bytes && (!p || ((uintptr_t)p & 255)))
          return report(PJRT_Error_Code_INVALID_ARGUMENT,
                        "output %d must be a non-null 256-byte aligned device pointer", sl.index);
        ptr[s] = p;
        break;
      }
      case Slot::CONSTANT:
        ptr[s] = exe.constants[s]->ptr;
        break;
      case Slot::TEMP:
        ptr[s] = base + off;
        off += (bytes + 255) & ~(size_t)255;
        break;
    }
  }
  // the caller's current device is put back on every return path
  int prev = -1;
  if (hipGetDevice(&prev) != hipSuccess) return report(PJRT_Error_Code_INTERNAL, "cannot read the current device");
  struct RestoreDevice {
    int dev;
    ~RestoreDevice() { (void)hipSetDevice(dev); }
  } restore{prev};
  try {
    std::lock_guard<std::recursive_mutex> lk(d->launch_mu);
    if (hipSetDevice(d->hip_ordinal) != hipSuccess)
      return report(PJRT_Error_Code_INTERNAL, "cannot make device %d current", d->hip_ordinal);
    // (never timed, not even for a started profiler session: timing creates events)
    enqueue_steps(le->client, plan, ptr, (hipStream_t)stream, nullptr, false, d->id, false);
  } catch (const Status& st) {
    return report(st.code, "%s", st.what());
  }
  return 0;
}
