// The PJRT profiler extension (crates/ryft-pjrt/src/extensions/profiler.rs:152-230, its C structs at :380-520):
// Create / Start / Stop / CollectData / Destroy, results as a serialized XSpace (the XPlane protobuf of TSL's
// profiler, fields per crates/ryft-xla-sys/src/protos.rs:3574-3810).
//
// A session records, while started, every kernel step any client of the process enqueues (the HIP events its first
// and last launch record) and the host span of each execution. Stop waits for the recorded steps, turns their events
// into times and releases them, so a stopped session holds no HIP object; the session registry is touched only by
// the calling threads of execute and of the profiler entry points (never by a client's completion worker or at
// process exit).
#include <hip/hip_runtime_api.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "runtime.h"

namespace ryft {

int64_t wall_clock_ns() {
  return std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::system_clock::now().time_since_epoch())
      .count();
}

namespace {

struct HostSpan {
  std::string name;
  int64_t begin_ns, end_ns;
};

struct DeviceEvent {  // a step after Stop: times relative to the first recorded step of its device
  std::string name;
  int device;
  int64_t host_ns;
  double offset_ms, duration_ms, flops, bytes;
};

struct Session {
  enum State { CREATED, STARTED, STOPPED } state = CREATED;
  uint32_t host_level = 2, device_level = 1;  // ProfileOptions.host_tracing_level / device_tracing_level
  std::mutex mu;
  std::vector<StepTiming> steps;  // while started
  std::vector<HostSpan> host;
  std::vector<DeviceEvent> device;  // after Stop
  std::vector<std::string> errors;
  std::string xspace;  // serialized results (CollectData), NUL-terminated
};

std::mutex g_mu;
std::vector<Session*> g_started;
std::atomic<int> g_started_count{0};

// ---------------------------------------------------------------- protobuf writer (proto3 wire format)
struct Pb {
  std::string out;
  void varint(uint64_t v) {
    do {
      uint8_t b = v & 0x7f;
      v >>= 7;
      out.push_back((char)(b | (v ? 0x80 : 0)));
    } while (v);
  }
  void key(int field, int wire) { varint(((uint64_t)field << 3) | (uint64_t)wire); }
  void i64(int field, int64_t v) {
    if (!v) return;
    key(field, 0);
    varint((uint64_t)v);
  }
  void dbl(int field, double v) {
    key(field, 1);
    char b[8];
    memcpy(b, &v, 8);
    out.append(b, 8);
  }
  void str(int field, const std::string& s) {
    if (s.empty()) return;
    key(field, 2);
    varint(s.size());
    out += s;
  }
  void msg(int field, const Pb& m) {
    key(field, 2);
    varint(m.out.size());
    out += m.out;
  }
};

// XEventMetadata {id 1, name 2, display_name 4}, XStatMetadata {id 1, name 2, description 3}; map entries {key 1,
// value 2}.
void event_metadata(Pb& plane, int64_t id, const std::string& name) {
  Pb md, entry;
  md.i64(1, id);
  md.str(2, name);
  md.str(4, name);
  entry.i64(1, id);
  entry.msg(2, md);
  plane.msg(4, entry);
}
void stat_metadata(Pb& plane, int64_t id, const std::string& name, const std::string& what) {
  Pb md, entry;
  md.i64(1, id);
  md.str(2, name);
  md.str(3, what);
  entry.i64(1, id);
  entry.msg(2, md);
  plane.msg(5, entry);
}
// XEvent {metadata_id 1, offset_ps 2, duration_ps 3, stats 4}; XStat {metadata_id 1, double_value 2}
Pb xevent(int64_t md, int64_t offset_ps, int64_t duration_ps, const std::vector<std::pair<int64_t, double>>& stats) {
  Pb e;
  e.i64(1, md);
  e.key(2, 0);
  e.varint((uint64_t)offset_ps);
  e.i64(3, duration_ps);
  for (auto& s : stats) {
    Pb st;
    st.i64(1, s.first);
    st.dbl(2, s.second);
    e.msg(4, st);
  }
  return e;
}

std::string serialize(const Session& s) {
  Pb space;
  int64_t plane_id = 0;
  // host plane: one line of execution spans
  if (s.host_level > 0) {
    Pb plane, line;
    plane.i64(1, plane_id++);
    plane.str(2, "/host:CPU");
    std::map<std::string, int64_t> md;
    const int64_t t0 = s.host.empty() ? 0 : s.host.front().begin_ns;
    line.i64(1, 1);
    line.str(2, "PJRT client");
    line.i64(3, t0);
    for (const HostSpan& h : s.host) {
      auto it = md.emplace(h.name, (int64_t)md.size() + 1).first;
      line.msg(4, xevent(it->second, (h.begin_ns - t0) * 1000, (h.end_ns - h.begin_ns) * 1000, {}));
    }
    if (!s.host.empty()) line.i64(9, (s.host.back().end_ns - t0) * 1000);
    plane.msg(3, line);
    for (auto& m : md) event_metadata(plane, m.second, m.first);
    space.msg(1, plane);
  }
  // one plane per device that ran steps: a line of kernel steps on the device stream, times from HIP events
  if (s.device_level > 0) {
    std::map<int, std::vector<const DeviceEvent*>> by_dev;
    for (const DeviceEvent& e : s.device) by_dev[e.device].push_back(&e);
    for (auto& dv : by_dev) {
      Pb plane, line;
      plane.i64(1, plane_id++);
      plane.str(2, "/device:GPU:" + std::to_string(dv.first));
      std::map<std::string, int64_t> md;
      line.i64(1, 1);
      line.str(2, "Stream #0");
      line.str(11, "Kernels");
      line.i64(3, dv.second.front()->host_ns);
      double end_ms = 0;
      for (const DeviceEvent* e : dv.second) {
        auto it = md.emplace(e->name, (int64_t)md.size() + 1).first;
        line.msg(4, xevent(it->second, (int64_t)(e->offset_ms * 1e9), (int64_t)(e->duration_ms * 1e9),
                           {{1, e->flops}, {2, e->bytes}}));
        end_ms = std::max(end_ms, e->offset_ms + e->duration_ms);
      }
      line.i64(9, (int64_t)(end_ms * 1e9));
      plane.msg(3, line);
      for (auto& m : md) event_metadata(plane, m.second, m.first);
      stat_metadata(plane, 1, "flops", "algorithmic floating-point / integer operations of the step");
      stat_metadata(plane, 2, "bytes accessed", "algorithmic bytes read and written by the step");
      space.msg(1, plane);
    }
  }
  for (const std::string& e : s.errors) space.str(2, e);
  char host[256] = {0};
  if (gethostname(host, sizeof(host) - 1) == 0 && host[0]) space.str(4, host);
  return space.out;
}

// ProfileOptions (protos.rs:3423-3490): host_tracing_level 2, device_tracing_level 3, version 5 (uint32); other fields
// skipped. As in TSL's profiler, options of version 0 stand for the default session (host level 2, device level 1).
void decode_options(const char* p, size_t n, Session* s) {
  uint32_t version = 0, host = 0, device = 0;
  const uint8_t* q = (const uint8_t*)p;
  const uint8_t* end = q + n;
  auto varint = [&]() -> uint64_t {
    uint64_t v = 0;
    for (int shift = 0; shift < 64; shift += 7) {
      if (q >= end) invalid("malformed profile options: truncated varint");
      const uint8_t b = *q++;
      v |= (uint64_t)(b & 0x7f) << shift;
      if (!(b & 0x80)) return v;
    }
    invalid("malformed profile options: varint too long");
  };
  while (q < end) {
    const uint64_t k = varint();
    const int field = (int)(k >> 3), wire = (int)(k & 7);
    if (wire == 0) {
      const uint64_t v = varint();
      if (field == 2) host = (uint32_t)v;
      if (field == 3) device = (uint32_t)v;
      if (field == 5) version = (uint32_t)v;
    } else if (wire == 2) {
      const uint64_t len = varint();
      if (len > (uint64_t)(end - q)) invalid("malformed profile options: field runs past the end");
      q += len;
    } else if (wire == 1 || wire == 5) {
      const size_t w = wire == 1 ? 8 : 4;
      if ((size_t)(end - q) < w) invalid("malformed profile options: truncated fixed field");
      q += w;
    } else {
      invalid("malformed profile options: wire type " + std::to_string(wire));
    }
  }
  if (version) {
    s->host_level = host;
    s->device_level = device;
  }
}

void unregister(Session* s) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = std::find(g_started.begin(), g_started.end(), s);
  if (it != g_started.end()) {
    g_started.erase(it);
    g_started_count.fetch_sub(1);
  }
}

}  // namespace

bool profiler_sessions_active() { return g_started_count.load(std::memory_order_relaxed) > 0; }

void profiler_record_step(const StepTiming& t) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (Session* s : g_started) {
    std::lock_guard<std::mutex> sl(s->mu);
    s->steps.push_back(t);
  }
}

void profiler_record_host(const std::string& name, int64_t begin_ns, int64_t end_ns) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (Session* s : g_started) {
    std::lock_guard<std::mutex> sl(s->mu);
    s->host.push_back({name, begin_ns, end_ns});
  }
}

}  // namespace ryft

// ------------------------------------------------------------------------------------------------ C entry points
using namespace ryft;

namespace {

PLUGIN_Profiler_Error* prof_error(PJRT_Error_Code code, const std::string& msg) {
  return reinterpret_cast<PLUGIN_Profiler_Error*>(new Status(code, msg));
}
Session* session(PLUGIN_Profiler* p) { return reinterpret_cast<Session*>(p); }

#define PROF_TRY try {
#define PROF_CATCH                                                                              \
  }                                                                                             \
  catch (const Status& st) { return prof_error(st.code, st.what()); }                           \
  catch (const std::exception& ex) { return prof_error(PJRT_Error_Code_INTERNAL, ex.what()); } \
  return nullptr;

void Prof_Error_Destroy(PLUGIN_Profiler_Error_Destroy_Args* args) {
  if (args) delete reinterpret_cast<Status*>(args->error);
}
void Prof_Error_Message(PLUGIN_Profiler_Error_Message_Args* args) {
  if (!args || !args->error) return;
  const Status* s = reinterpret_cast<const Status*>(args->error);
  args->message = s->what();
  args->message_size = strlen(s->what());
}
PLUGIN_Profiler_Error* Prof_Error_GetCode(PLUGIN_Profiler_Error_GetCode_Args* args) {
  if (!args || !args->error) return prof_error(PJRT_Error_Code_INVALID_ARGUMENT, "error is null");
  args->code = (int)reinterpret_cast<const Status*>(args->error)->code;
  return nullptr;
}

PLUGIN_Profiler_Error* Prof_Create(PLUGIN_Profiler_Create_Args* args) {
  if (!args) return prof_error(PJRT_Error_Code_INVALID_ARGUMENT, "args is null");
  PROF_TRY
  auto s = std::make_unique<Session>();
  if (args->options && args->options_size) decode_options(args->options, args->options_size, s.get());
  args->profiler = reinterpret_cast<PLUGIN_Profiler*>(s.release());
  PROF_CATCH
}

PLUGIN_Profiler_Error* Prof_Destroy(PLUGIN_Profiler_Destroy_Args* args) {
  if (!args || !args->profiler) return prof_error(PJRT_Error_Code_INVALID_ARGUMENT, "profiler is null");
  Session* s = session(args->profiler);
  unregister(s);
  delete s;  // a session destroyed while started releases its recorded steps' events here
  return nullptr;
}

PLUGIN_Profiler_Error* Prof_Start(PLUGIN_Profiler_Start_Args* args) {
  if (!args || !args->profiler) return prof_error(PJRT_Error_Code_INVALID_ARGUMENT, "profiler is null");
  Session* s = session(args->profiler);
  std::lock_guard<std::mutex> lk(g_mu);
  if (s->state != Session::CREATED)
    return prof_error(PJRT_Error_Code_FAILED_PRECONDITION, "the profiler has already been started");
  s->state = Session::STARTED;
  g_started.push_back(s);
  g_started_count.fetch_add(1);
  return nullptr;
}

PLUGIN_Profiler_Error* Prof_Stop(PLUGIN_Profiler_Stop_Args* args) {
  if (!args || !args->profiler) return prof_error(PJRT_Error_Code_INVALID_ARGUMENT, "profiler is null");
  Session* s = session(args->profiler);
  {
    std::lock_guard<std::mutex> lk(g_mu);
    if (s->state != Session::STARTED)
      return prof_error(PJRT_Error_Code_FAILED_PRECONDITION, "the profiler is not started");
  }
  unregister(s);  // no step is recorded into it from here on
  std::vector<StepTiming> steps;
  {
    std::lock_guard<std::mutex> sl(s->mu);
    steps.swap(s->steps);
    s->state = Session::STOPPED;
  }
  // the steps' times: wait for each step, then measure it and place it after the first step of its device
  std::map<int, const StepTiming*> first;
  for (const StepTiming& t : steps)
    if (!first.count(t.device)) first[t.device] = &t;
  for (const StepTiming& t : steps) {
    float dur = 0, off = 0;
    hipError_t e = hipEventSynchronize(t.ev->stop);
    if (e == hipSuccess) e = hipEventElapsedTime(&dur, t.ev->start, t.ev->stop);
    if (e == hipSuccess) e = hipEventElapsedTime(&off, first[t.device]->ev->start, t.ev->start);
    if (e != hipSuccess) {
      s->errors.push_back("step " + t.name + ": " + hipGetErrorString(e));
      continue;
    }
    s->device.push_back({t.name, t.device, first[t.device]->host_ns, (double)off, (double)dur, t.flops, t.bytes});
  }
  steps.clear();  // releases the events (the last holder destroys them)
  return nullptr;
}

PLUGIN_Profiler_Error* Prof_CollectData(PLUGIN_Profiler_CollectData_Args* args) {
  if (!args || !args->profiler) return prof_error(PJRT_Error_Code_INVALID_ARGUMENT, "profiler is null");
  Session* s = session(args->profiler);
  if (args->buffer) return nullptr;  // the results were handed out by the first call
  PROF_TRY
  std::lock_guard<std::mutex> sl(s->mu);
  if (s->state != Session::STOPPED)
    return prof_error(PJRT_Error_Code_FAILED_PRECONDITION, "stop the profiler before collecting its data");
  // as XLA's plugins do: one call with a null buffer serializes into storage the session owns, NUL-terminated, and
  // reports its size including the terminator
  s->xspace = serialize(*s);
  s->xspace.push_back('\0');
  args->buffer = (uint8_t*)&s->xspace[0];
  args->buffer_size_in_bytes = s->xspace.size();
  PROF_CATCH
}

PLUGIN_Profiler_Api g_profiler_api = {
    sizeof(PLUGIN_Profiler_Api), nullptr,      Prof_Error_Destroy, Prof_Error_Message, Prof_Error_GetCode,
    Prof_Create,                 Prof_Destroy, Prof_Start,         Prof_Stop,          Prof_CollectData,
};

}  // namespace

namespace ryft {
PJRT_Profiler_Extension g_profiler_extension = {
    {sizeof(PJRT_Profiler_Extension), PJRT_Extension_Type_Profiler, nullptr},
    &g_profiler_api,
    0,
};
}  // namespace ryft
