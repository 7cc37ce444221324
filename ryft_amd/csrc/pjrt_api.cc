// The PJRT C API table exported through GetPjrtApi(). Each entry validates its *_Args struct, converts C++
// exceptions into PJRT_Error objects, and forwards to the runtime. Call contracts follow ryft-pjrt:
//   error objects are read then destroyed by the caller (crates/ryft-pjrt/src/errors.rs:76-180);
//   an unimplemented slot is left null (macros.rs:92-96);
//   LoadedExecutable_GetExecutable hands out a fresh handle the caller destroys after each execute
//   (programs.rs:915, 426-432);
//   ToHostBuffer with dst == null only reports dst_size (buffers.rs:1242-1253).
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstddef>
#include <cstring>
#include <mutex>
#include <string>

#include "mlir_common.h"
#include "ryft_mi355x.h"
#include "runtime.h"

namespace ryft {

struct ErrorObj {
  PJRT_Error_Code code;
  std::string message;
  Payload payload;
};

PJRT_Error* make_pjrt_error(PJRT_Error_Code code, const std::string& msg, const Payload& payload) {
  return reinterpret_cast<PJRT_Error*>(new ErrorObj{code, msg, payload});
}

}  // namespace ryft

using namespace ryft;

namespace {

template <typename T, typename H>
T* from(H* h) { return reinterpret_cast<T*>(h); }
template <typename H, typename T>
H* to(T* p) { return reinterpret_cast<H*>(p); }

#define API_TRY try {
#define API_CATCH                                                                 \
  }                                                                               \
  catch (const Status& s) { return make_pjrt_error(s.code, s.what(), s.payload); }\
  catch (const std::bad_alloc&) {                                                 \
    return make_pjrt_error(PJRT_Error_Code_RESOURCE_EXHAUSTED, "host allocation failed"); \
  }                                                                               \
  catch (const std::exception& e) { return make_pjrt_error(PJRT_Error_Code_INTERNAL, e.what()); } \
  return nullptr;

// The caller's struct must at least reach the last field this entry point touches.
#define NEED_ARGS(Type, field)                                                                                   \
  do {                                                                                                           \
    if (!args || args->struct_size < offsetof(Type, field) + sizeof(((Type*)nullptr)->field))                    \
      return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, #Type ": struct_size is too small");              \
  } while (0)

#define NEED(ptr, what) \
  do {                  \
    if (!(ptr)) return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, what " is null"); \
  } while (0)

// ------------------------------------------------------------------------------------------------ errors
void Error_Destroy(PJRT_Error_Destroy_Args* args) {
  if (args && args->error) delete from<ErrorObj>(args->error);
}
void Error_Message(PJRT_Error_Message_Args* args) {
  const ErrorObj* e = reinterpret_cast<const ErrorObj*>(args->error);
  args->message = e ? e->message.c_str() : "";
  args->message_size = e ? e->message.size() : 0;
}
PJRT_Error* Error_GetCode(PJRT_Error_GetCode_Args* args) {
  NEED_ARGS(PJRT_Error_GetCode_Args, code);
  const ErrorObj* e = reinterpret_cast<const ErrorObj*>(args->error);
  args->code = e ? e->code : PJRT_Error_Code_OK;
  return nullptr;
}
PJRT_Error* Error_ForEachPayload(PJRT_Error_ForEachPayload_Args* args) {
  NEED_ARGS(PJRT_Error_ForEachPayload_Args, user_arg);
  const ErrorObj* e = reinterpret_cast<const ErrorObj*>(args->error);
  if (!e || e->payload.empty()) return nullptr;
  NEED(args->visitor, "visitor");
  for (const auto& kv : e->payload)
    args->visitor(kv.first.data(), kv.first.size(), kv.second.data(), kv.second.size(), args->user_arg);
  return nullptr;
}

// ------------------------------------------------------------------------------------------------ plugin
struct PluginAttributes {
  int64_t current[3] = {1, 16, 0};
  int64_t minimum[3] = {0, 9, 0};
  std::string version = "0.1.0";
  std::vector<PJRT_NamedValue> values;
  PluginAttributes() {
    auto list = [](const char* name, const int64_t* v) {
      PJRT_NamedValue n{};
      n.struct_size = sizeof(PJRT_NamedValue);
      n.name = name;
      n.name_size = strlen(name);
      n.type = PJRT_NamedValue_kInt64List;
      n.int64_array_value = v;
      n.value_size = 3;
      return n;
    };
    values.push_back(list("stablehlo_current_version", current));
    values.push_back(list("stablehlo_minimum_version", minimum));
    PJRT_NamedValue x{};
    x.struct_size = sizeof(PJRT_NamedValue);
    x.name = "xla_version";
    x.name_size = 11;
    x.type = PJRT_NamedValue_kInt64;
    x.int64_value = 2;
    x.value_size = 1;
    values.push_back(x);
    PJRT_NamedValue v{};
    v.struct_size = sizeof(PJRT_NamedValue);
    v.name = "ryft_mi355x_version";
    v.name_size = strlen(v.name);
    v.type = PJRT_NamedValue_kString;
    v.string_value = version.c_str();
    v.value_size = version.size();
    values.push_back(v);
  }
};
PluginAttributes& plugin_attributes() {
  static PluginAttributes a;
  return a;
}

PJRT_Error* Plugin_Initialize(PJRT_Plugin_Initialize_Args* args) {
  NEED_ARGS(PJRT_Plugin_Initialize_Args, extension_start);
  return nullptr;
}
PJRT_Error* Plugin_Attributes(PJRT_Plugin_Attributes_Args* args) {
  NEED_ARGS(PJRT_Plugin_Attributes_Args, num_attributes);
  auto& a = plugin_attributes();
  args->attributes = a.values.data();
  args->num_attributes = a.values.size();
  return nullptr;
}

// ------------------------------------------------------------------------------------------------ events
PJRT_Event* wrap_event(const EventPtr& e) { return to<PJRT_Event>(new Event{e}); }

PJRT_Error* Event_Destroy(PJRT_Event_Destroy_Args* args) {
  NEED_ARGS(PJRT_Event_Destroy_Args, event);
  delete from<Event>(args->event);
  return nullptr;
}
PJRT_Error* Event_IsReady(PJRT_Event_IsReady_Args* args) {
  NEED_ARGS(PJRT_Event_IsReady_Args, is_ready);
  NEED(args->event, "event");
  API_TRY
  args->is_ready = from<Event>(args->event)->state->poll();
  API_CATCH
}
PJRT_Error* Event_Error(PJRT_Event_Error_Args* args) {
  NEED_ARGS(PJRT_Event_Error_Args, event);
  NEED(args->event, "event");
  auto& st = from<Event>(args->event)->state;
  std::lock_guard<std::mutex> lk(st->mu);
  if (!st->ready) return make_pjrt_error(PJRT_Error_Code_FAILED_PRECONDITION, "event is not ready");
  return st->code == PJRT_Error_Code_OK ? nullptr : make_pjrt_error(st->code, st->message, st->payload);
}
PJRT_Error* Event_Await(PJRT_Event_Await_Args* args) {
  NEED_ARGS(PJRT_Event_Await_Args, event);
  NEED(args->event, "event");
  API_TRY
  auto& st = from<Event>(args->event)->state;
  st->wait();
  std::lock_guard<std::mutex> lk(st->mu);
  if (st->code != PJRT_Error_Code_OK) return make_pjrt_error(st->code, st->message, st->payload);
  API_CATCH
}
PJRT_Error* Event_OnReady(PJRT_Event_OnReady_Args* args) {
  NEED_ARGS(PJRT_Event_OnReady_Args, user_arg);
  NEED(args->event, "event");
  NEED(args->callback, "callback");
  auto st = from<Event>(args->event)->state;
  bool run_now = false, hand_to_worker = false;
  {
    std::lock_guard<std::mutex> lk(st->mu);
    if (st->ready) {
      run_now = true;
    } else {
      st->callbacks.push_back({args->callback, args->user_arg});
      hand_to_worker = st->lazy_owner && !st->queued;
      st->queued |= hand_to_worker;
    }
  }
  if (hand_to_worker) st->lazy_owner->enqueue_completion(st);
  if (run_now) {
    // each callback receives its own error object; the callee destroys it (events.rs:100-108)
    args->callback(st->code == PJRT_Error_Code_OK ? nullptr : make_pjrt_error(st->code, st->message), args->user_arg);
  }
  return nullptr;
}
PJRT_Error* Event_Create(PJRT_Event_Create_Args* args) {
  NEED_ARGS(PJRT_Event_Create_Args, event);
  args->event = wrap_event(std::make_shared<EventState>());
  return nullptr;
}
PJRT_Error* Event_Set(PJRT_Event_Set_Args* args) {
  NEED_ARGS(PJRT_Event_Set_Args, error_message_size);
  NEED(args->event, "event");
  auto& st = from<Event>(args->event)->state;
  {
    std::lock_guard<std::mutex> lk(st->mu);
    if (st->ready) return make_pjrt_error(PJRT_Error_Code_FAILED_PRECONDITION, "event is already set");
  }
  st->set_ready(args->error_code,
                args->error_message ? std::string(args->error_message, args->error_message_size) : std::string());
  return nullptr;
}

// ------------------------------------------------------------------------------------------------ client
std::mutex g_client_mu;

PJRT_Error* Client_Create(PJRT_Client_Create_Args* args) {
  NEED_ARGS(PJRT_Client_Create_Args, client);
  API_TRY
  // Recognised options: visible_devices (int64 list, as GpuClientOptions, clients.rs:453-573) and compile_only
  // (bool, plugin-specific: plans are built but nothing runs), fast_paths (bool, plugin-specific, default true:
  // false runs every row-fused step through the interpreted kernel, for cross-checks). Others are ignored.
  std::vector<int> visible;
  bool compile_only = false, fast_paths = true;
  for (size_t i = 0; i < args->num_options; ++i) {
    const PJRT_NamedValue& o = args->create_options[i];
    std::string name(o.name, o.name_size);
    if (name == "visible_devices" && o.type == PJRT_NamedValue_kInt64List)
      for (size_t k = 0; k < o.value_size; ++k) visible.push_back((int)o.int64_array_value[k]);
    if (name == "compile_only" && o.type == PJRT_NamedValue_kBool) compile_only = o.bool_value;
    if (name == "fast_paths" && o.type == PJRT_NamedValue_kBool) fast_paths = o.bool_value;
  }
  std::lock_guard<std::mutex> lk(g_client_mu);
  Client* c = new Client(visible, compile_only);
  c->fast_paths = fast_paths;
  args->client = to<PJRT_Client>(c);
  API_CATCH
}
PJRT_Error* Client_Destroy(PJRT_Client_Destroy_Args* args) {
  NEED_ARGS(PJRT_Client_Destroy_Args, client);
  API_TRY
  std::lock_guard<std::mutex> lk(g_client_mu);
  delete from<Client>(args->client);
  API_CATCH
}
PJRT_Error* Client_PlatformName(PJRT_Client_PlatformName_Args* args) {
  NEED_ARGS(PJRT_Client_PlatformName_Args, platform_name_size);
  NEED(args->client, "client");
  Client* c = from<Client>(args->client);
  args->platform_name = c->platform_name.c_str();
  args->platform_name_size = c->platform_name.size();
  return nullptr;
}
PJRT_Error* Client_ProcessIndex(PJRT_Client_ProcessIndex_Args* args) {
  NEED_ARGS(PJRT_Client_ProcessIndex_Args, process_index);
  args->process_index = 0;
  return nullptr;
}
PJRT_Error* Client_PlatformVersion(PJRT_Client_PlatformVersion_Args* args) {
  NEED_ARGS(PJRT_Client_PlatformVersion_Args, platform_version_size);
  NEED(args->client, "client");
  Client* c = from<Client>(args->client);
  args->platform_version = c->platform_version.c_str();
  args->platform_version_size = c->platform_version.size();
  return nullptr;
}
PJRT_Error* Client_Devices(PJRT_Client_Devices_Args* args) {
  NEED_ARGS(PJRT_Client_Devices_Args, num_devices);
  NEED(args->client, "client");
  Client* c = from<Client>(args->client);
  args->devices = reinterpret_cast<PJRT_Device* const*>(c->device_ptrs.data());
  args->num_devices = c->device_ptrs.size();
  return nullptr;
}
PJRT_Error* Client_AddressableDevices(PJRT_Client_AddressableDevices_Args* args) {
  NEED_ARGS(PJRT_Client_AddressableDevices_Args, num_addressable_devices);
  NEED(args->client, "client");
  Client* c = from<Client>(args->client);
  args->addressable_devices = reinterpret_cast<PJRT_Device* const*>(c->device_ptrs.data());
  args->num_addressable_devices = c->device_ptrs.size();
  return nullptr;
}
PJRT_Error* Client_LookupDevice(PJRT_Client_LookupDevice_Args* args) {
  NEED_ARGS(PJRT_Client_LookupDevice_Args, device);
  NEED(args->client, "client");
  Client* c = from<Client>(args->client);
  if (args->id < 0 || args->id >= (int)c->device_ptrs.size())
    return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, "no device with id " + std::to_string(args->id));
  args->device = to<PJRT_Device>(c->device_ptrs[args->id]);
  return nullptr;
}
PJRT_Error* Client_LookupAddressableDevice(PJRT_Client_LookupAddressableDevice_Args* args) {
  NEED_ARGS(PJRT_Client_LookupAddressableDevice_Args, addressable_device);
  NEED(args->client, "client");
  Client* c = from<Client>(args->client);
  if (args->local_hardware_id < 0 || args->local_hardware_id >= (int)c->device_ptrs.size())
    return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT,
                           "no addressable device with local hardware id " + std::to_string(args->local_hardware_id));
  args->addressable_device = to<PJRT_Device>(c->device_ptrs[args->local_hardware_id]);
  return nullptr;
}
PJRT_Error* Client_AddressableMemories(PJRT_Client_AddressableMemories_Args* args) {
  NEED_ARGS(PJRT_Client_AddressableMemories_Args, num_addressable_memories);
  NEED(args->client, "client");
  Client* c = from<Client>(args->client);
  args->addressable_memories = reinterpret_cast<PJRT_Memory* const*>(c->memory_ptrs.data());
  args->num_addressable_memories = c->memory_ptrs.size();
  return nullptr;
}
// One replica, one partition, on the client's first device (none on a compile-only client).
LoadedExecutable* load_executable(Client* c, std::shared_ptr<Executable> exe) {
  auto le = new LoadedExecutable();
  le->client = c;
  le->exe = std::move(exe);
  if (!c->device_ptrs.empty()) {
    le->devices = {c->device_ptrs.at(le->exe->device_index)};
    le->logical_ids = {PJRT_LogicalDeviceIds{0, 0}};
  }
  return le;
}

PJRT_Error* Client_Compile(PJRT_Client_Compile_Args* args) {
  NEED_ARGS(PJRT_Client_Compile_Args, executable);
  NEED(args->client, "client");
  NEED(args->program, "program");
  API_TRY
  Client* c = from<Client>(args->client);
  const PJRT_Program* p = args->program;
  std::string format = p->format ? std::string(p->format, p->format_size) : std::string("mlir");
  std::string code(p->code ? p->code : "", p->code ? p->code_size : 0);
  std::string opts(args->compile_options ? args->compile_options : "", args->compile_options ? args->compile_options_size : 0);
  args->executable = to<PJRT_LoadedExecutable>(load_executable(c, compile_program(c, code, format, opts)));
  API_CATCH
}
PJRT_Error* Client_DefaultDeviceAssignment(PJRT_Client_DefaultDeviceAssignment_Args* args) {
  NEED_ARGS(PJRT_Client_DefaultDeviceAssignment_Args, default_assignment);
  NEED(args->client, "client");
  Client* c = from<Client>(args->client);
  int64_t need = (int64_t)args->num_replicas * args->num_partitions;
  if (need > (int64_t)c->device_ptrs.size())
    return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT,
                           "requested " + std::to_string(need) + " devices but only " + std::to_string(c->device_ptrs.size()) + " exist");
  if ((int64_t)args->default_assignment_size < need)
    return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, "default_assignment is too small");
  for (int64_t i = 0; i < need; ++i) args->default_assignment[i] = (int)i;
  return nullptr;
}

Device* device_for(Client* c, PJRT_Device* device, PJRT_Memory* memory) {
  if (device) return from<Device>(device);
  if (memory) return from<Memory>(memory)->devices.at(0);
  return c->device_ptrs.at(0);
}

PJRT_Error* Client_BufferFromHostBuffer(PJRT_Client_BufferFromHostBuffer_Args* args) {
  NEED_ARGS(PJRT_Client_BufferFromHostBuffer_Args, buffer);
  NEED(args->client, "client");
  API_TRY
  Client* c = from<Client>(args->client);
  DType t;
  if (!dtype_from_pjrt(args->type, &t))
    return make_pjrt_error(PJRT_Error_Code_UNIMPLEMENTED, "buffer element type " + std::to_string(args->type) + " is not supported");
  if (args->device_layout && !(args->device_layout->type == PJRT_Buffer_MemoryLayout_Type_Tiled &&
                               args->device_layout->tiled.num_tiles == 0)) {
    // only the default dense row-major device layout is supported
    bool ok = args->device_layout->type == PJRT_Buffer_MemoryLayout_Type_Tiled;
    if (!ok) return make_pjrt_error(PJRT_Error_Code_UNIMPLEMENTED, "custom device layouts are not supported");
  }
  std::vector<int64_t> dims(args->dims, args->dims + args->num_dims);
  Device* d = device_for(c, args->device, args->memory);
  EventPtr done;
  Buffer* b = buffer_from_host(c, d, args->data, t, dims, args->byte_strides, args->num_byte_strides, &done);
  args->buffer = to<PJRT_Buffer>(b);
  args->done_with_host_buffer = wrap_event(done);
  API_CATCH
}
PJRT_Error* Client_CreateUninitializedBuffer(PJRT_Client_CreateUninitializedBuffer_Args* args) {
  NEED_ARGS(PJRT_Client_CreateUninitializedBuffer_Args, buffer);
  NEED(args->client, "client");
  API_TRY
  Client* c = from<Client>(args->client);
  DType t;
  if (!dtype_from_pjrt(args->shape_element_type, &t))
    return make_pjrt_error(PJRT_Error_Code_UNIMPLEMENTED, "unsupported element type");
  auto b = new Buffer();
  b->client = c;
  b->device = device_for(c, args->device, args->memory);
  b->dtype = t;
  b->dims.assign(args->shape_dims, args->shape_dims + args->shape_num_dims);
  for (int i = (int)b->dims.size() - 1; i >= 0; --i) b->minor_to_major.push_back(i);
  b->mem = c->allocate(b->device, b->bytes());
  auto e = std::make_shared<EventState>();
  e->ready = true;
  b->ready = e;
  args->buffer = to<PJRT_Buffer>(b);
  API_CATCH
}

// (name, value) payload strings from PJRT_NamedValues; non-string values are printed in decimal
Payload payload_from(const PJRT_NamedValue* v, size_t n) {
  Payload out;
  if (n && !v) invalid("payload is null");
  for (size_t i = 0; i < n; ++i) {
    if (v[i].name_size && !v[i].name) invalid("payload name is null");
    std::string name(v[i].name ? v[i].name : "", v[i].name_size), value;
    switch (v[i].type) {
      case PJRT_NamedValue_kString:
        if (v[i].value_size && !v[i].string_value) invalid("payload value is null");
        value.assign(v[i].string_value ? v[i].string_value : "", v[i].value_size);
        break;
      case PJRT_NamedValue_kInt64: value = std::to_string(v[i].int64_value); break;
      case PJRT_NamedValue_kFloat: value = std::to_string(v[i].float_value); break;
      case PJRT_NamedValue_kBool: value = v[i].bool_value ? "true" : "false"; break;
      case PJRT_NamedValue_kInt64List:
        for (size_t k = 0; k < v[i].value_size; ++k)
          value += (k ? "," : "") + std::to_string(v[i].int64_array_value[k]);
        break;
      default: invalid("payload value of unknown type " + std::to_string((int)v[i].type));
    }
    out.emplace_back(std::move(name), std::move(value));
  }
  return out;
}

// The error a caller hands in (message bytes, code, payload), checked to be an error.
Status caller_error(PJRT_Error_Code code, const char* msg, size_t msg_size, const PJRT_NamedValue* payload,
                    size_t payload_size) {
  if (code == PJRT_Error_Code_OK) invalid("error code is OK");
  if (msg_size && !msg) invalid("error message is null");
  return Status(code, std::string(msg ? msg : "", msg_size), payload_from(payload, payload_size));
}

PJRT_Error* Client_CreateErrorBuffer(PJRT_Client_CreateErrorBuffer_Args* args) {
  NEED_ARGS(PJRT_Client_CreateErrorBuffer_Args, buffer);
  NEED(args->client, "client");
  NEED(args->memory, "memory");
  API_TRY
  Client* c = from<Client>(args->client);
  // the payload fields follow `buffer`: a caller's older, shorter struct has none
  const bool has_payload = args->struct_size >= offsetof(PJRT_Client_CreateErrorBuffer_Args, payload_size) +
                                                     sizeof(args->payload_size);
  Status err = caller_error(args->error_code, args->error_message, args->error_message_size,
                            has_payload ? args->payload : nullptr, has_payload ? args->payload_size : 0);
  DType t;
  if (!dtype_from_pjrt(args->shape_element_type, &t))
    return make_pjrt_error(PJRT_Error_Code_UNIMPLEMENTED, "unsupported element type");
  if (args->shape_num_dims && !args->shape_dims) invalid("shape_dims is null");
  if (args->shape_layout && !(args->shape_layout->type == PJRT_Buffer_MemoryLayout_Type_Tiled &&
                              args->shape_layout->tiled.num_tiles == 0))
    return make_pjrt_error(PJRT_Error_Code_UNIMPLEMENTED, "custom device layouts are not supported");
  std::vector<int64_t> dims(args->shape_dims, args->shape_dims + args->shape_num_dims);
  check_tensor_shape(dims);
  auto b = std::make_unique<Buffer>();
  b->client = c;
  b->device = device_for(c, nullptr, args->memory);
  b->dtype = t;
  b->dims = std::move(dims);
  for (int i = (int)b->dims.size() - 1; i >= 0; --i) b->minor_to_major.push_back(i);
  b->ready = error_event(err);  // no device memory: every consumer fails with the error
  args->buffer = to<PJRT_Buffer>(b.release());
  API_CATCH
}

// ------------------------------------------------------------------------------------------------ devices
PJRT_Error* DeviceDescription_Id(PJRT_DeviceDescription_Id_Args* args) {
  NEED_ARGS(PJRT_DeviceDescription_Id_Args, id);
  NEED(args->device_description, "device_description");
  args->id = from<Device>(args->device_description)->id;
  return nullptr;
}
PJRT_Error* DeviceDescription_ProcessIndex(PJRT_DeviceDescription_ProcessIndex_Args* args) {
  NEED_ARGS(PJRT_DeviceDescription_ProcessIndex_Args, process_index);
  args->process_index = 0;
  return nullptr;
}
PJRT_Error* DeviceDescription_Attributes(PJRT_DeviceDescription_Attributes_Args* args) {
  NEED_ARGS(PJRT_DeviceDescription_Attributes_Args, attributes);
  NEED(args->device_description, "device_description");
  Device* d = from<Device>(args->device_description);
  args->attributes = d->attributes.data();
  args->num_attributes = d->attributes.size();
  return nullptr;
}
PJRT_Error* DeviceDescription_Kind(PJRT_DeviceDescription_Kind_Args* args) {
  NEED_ARGS(PJRT_DeviceDescription_Kind_Args, device_kind_size);
  NEED(args->device_description, "device_description");
  Device* d = from<Device>(args->device_description);
  args->device_kind = d->kind.c_str();
  args->device_kind_size = d->kind.size();
  return nullptr;
}
PJRT_Error* DeviceDescription_DebugString(PJRT_DeviceDescription_DebugString_Args* args) {
  NEED_ARGS(PJRT_DeviceDescription_DebugString_Args, debug_string_size);
  NEED(args->device_description, "device_description");
  Device* d = from<Device>(args->device_description);
  args->debug_string = d->debug.c_str();
  args->debug_string_size = d->debug.size();
  return nullptr;
}
PJRT_Error* DeviceDescription_ToString(PJRT_DeviceDescription_ToString_Args* args) {
  NEED_ARGS(PJRT_DeviceDescription_ToString_Args, to_string_size);
  NEED(args->device_description, "device_description");
  Device* d = from<Device>(args->device_description);
  args->to_string = d->to_string.c_str();
  args->to_string_size = d->to_string.size();
  return nullptr;
}
PJRT_Error* Device_GetDescription(PJRT_Device_GetDescription_Args* args) {
  NEED_ARGS(PJRT_Device_GetDescription_Args, device_description);
  NEED(args->device, "device");
  args->device_description = reinterpret_cast<PJRT_DeviceDescription*>(args->device);
  return nullptr;
}
PJRT_Error* Device_IsAddressable(PJRT_Device_IsAddressable_Args* args) {
  NEED_ARGS(PJRT_Device_IsAddressable_Args, is_addressable);
  args->is_addressable = true;
  return nullptr;
}
PJRT_Error* Device_LocalHardwareId(PJRT_Device_LocalHardwareId_Args* args) {
  NEED_ARGS(PJRT_Device_LocalHardwareId_Args, local_hardware_id);
  NEED(args->device, "device");
  args->local_hardware_id = from<Device>(args->device)->id;
  return nullptr;
}
PJRT_Error* Device_AddressableMemories(PJRT_Device_AddressableMemories_Args* args) {
  NEED_ARGS(PJRT_Device_AddressableMemories_Args, num_memories);
  NEED(args->device, "device");
  Device* d = from<Device>(args->device);
  args->memories = reinterpret_cast<PJRT_Memory* const*>(d->memories.data());
  args->num_memories = d->memories.size();
  return nullptr;
}
PJRT_Error* Device_DefaultMemory(PJRT_Device_DefaultMemory_Args* args) {
  NEED_ARGS(PJRT_Device_DefaultMemory_Args, memory);
  NEED(args->device, "device");
  args->memory = to<PJRT_Memory>(from<Device>(args->device)->default_memory);
  return nullptr;
}
PJRT_Error* Device_PoisonExecution(PJRT_Device_PoisonExecution_Args* args) {
  NEED_ARGS(PJRT_Device_PoisonExecution_Args, payload_size);
  NEED(args->device, "device");
  API_TRY
  Status err = caller_error(args->error_code, args->error_message, args->error_message_size, args->payload,
                            args->payload_size);
  args->poisoned = poison_execution(from<Device>(args->device), args->launch_id, err);
  API_CATCH
}
PJRT_Error* Device_MemoryStats(PJRT_Device_MemoryStats_Args* args) {
  NEED_ARGS(PJRT_Device_MemoryStats_Args, peak_pool_bytes_is_set);
  NEED(args->device, "device");
  Device* d = from<Device>(args->device);
  args->bytes_in_use = d->allocator->bytes_in_use();
  args->peak_bytes_in_use = d->allocator->peak_bytes();
  args->peak_bytes_in_use_is_set = true;
  args->num_allocs = d->allocator->num_allocs();
  args->num_allocs_is_set = true;
  size_t free_b = 0, total_b = 0;
  (void)hipSetDevice(d->hip_ordinal);
  if (hipMemGetInfo(&free_b, &total_b) == hipSuccess) {
    args->bytes_limit = (int64_t)total_b;
    args->bytes_limit_is_set = true;
  }
  return nullptr;
}

// ------------------------------------------------------------------------------------------------ memories
PJRT_Error* Memory_Id(PJRT_Memory_Id_Args* args) {
  NEED_ARGS(PJRT_Memory_Id_Args, id);
  NEED(args->memory, "memory");
  args->id = from<Memory>(args->memory)->id;
  return nullptr;
}
PJRT_Error* Memory_Kind(PJRT_Memory_Kind_Args* args) {
  NEED_ARGS(PJRT_Memory_Kind_Args, kind_size);
  NEED(args->memory, "memory");
  Memory* m = from<Memory>(args->memory);
  args->kind = m->kind.c_str();
  args->kind_size = m->kind.size();
  return nullptr;
}
// The id XLA's PJRT plugins report for the "device" memory kind (ryft-pjrt's memories.rs:354 pins it).
constexpr int kDeviceMemoryKindId = 42097224;

PJRT_Error* Memory_Kind_Id(PJRT_Memory_Kind_Id_Args* args) {
  NEED_ARGS(PJRT_Memory_Kind_Id_Args, kind_id);
  args->kind_id = kDeviceMemoryKindId;
  return nullptr;
}
PJRT_Error* Memory_DebugString(PJRT_Memory_DebugString_Args* args) {
  NEED_ARGS(PJRT_Memory_DebugString_Args, debug_string_size);
  NEED(args->memory, "memory");
  Memory* m = from<Memory>(args->memory);
  args->debug_string = m->debug.c_str();
  args->debug_string_size = m->debug.size();
  return nullptr;
}
PJRT_Error* Memory_ToString(PJRT_Memory_ToString_Args* args) {
  NEED_ARGS(PJRT_Memory_ToString_Args, to_string_size);
  NEED(args->memory, "memory");
  Memory* m = from<Memory>(args->memory);
  args->to_string = m->to_string.c_str();
  args->to_string_size = m->to_string.size();
  return nullptr;
}
PJRT_Error* Memory_AddressableByDevices(PJRT_Memory_AddressableByDevices_Args* args) {
  NEED_ARGS(PJRT_Memory_AddressableByDevices_Args, num_devices);
  NEED(args->memory, "memory");
  Memory* m = from<Memory>(args->memory);
  args->devices = reinterpret_cast<PJRT_Device* const*>(m->devices.data());
  args->num_devices = m->devices.size();
  return nullptr;
}

// ------------------------------------------------------------------------------------------------ executables
Executable& exe_of(PJRT_Executable* e) { return *from<ExecutableView>(e)->exe; }

PJRT_Error* Executable_Destroy(PJRT_Executable_Destroy_Args* args) {
  NEED_ARGS(PJRT_Executable_Destroy_Args, executable);
  delete from<ExecutableView>(args->executable);
  return nullptr;
}
PJRT_Error* Executable_Name(PJRT_Executable_Name_Args* args) {
  NEED_ARGS(PJRT_Executable_Name_Args, executable_name_size);
  NEED(args->executable, "executable");
  auto& e = exe_of(args->executable);
  args->executable_name = e.name.c_str();
  args->executable_name_size = e.name.size();
  return nullptr;
}
PJRT_Error* Executable_NumReplicas(PJRT_Executable_NumReplicas_Args* args) {
  NEED_ARGS(PJRT_Executable_NumReplicas_Args, num_replicas);
  args->num_replicas = 1;
  return nullptr;
}
PJRT_Error* Executable_NumPartitions(PJRT_Executable_NumPartitions_Args* args) {
  NEED_ARGS(PJRT_Executable_NumPartitions_Args, num_partitions);
  args->num_partitions = 1;
  return nullptr;
}
PJRT_Error* Executable_NumOutputs(PJRT_Executable_NumOutputs_Args* args) {
  NEED_ARGS(PJRT_Executable_NumOutputs_Args, num_outputs);
  NEED(args->executable, "executable");
  args->num_outputs = exe_of(args->executable).output_types.size();
  return nullptr;
}
PJRT_Error* Executable_SizeOfGeneratedCodeInBytes(PJRT_Executable_SizeOfGeneratedCodeInBytes_Args* args) {
  NEED_ARGS(PJRT_Executable_SizeOfGeneratedCodeInBytes_Args, size_in_bytes);
  args->size_in_bytes = 0;  // kernels are precompiled into the plugin
  return nullptr;
}
PJRT_Error* Executable_GetCostAnalysis(PJRT_Executable_GetCostAnalysis_Args* args) {
  NEED_ARGS(PJRT_Executable_GetCostAnalysis_Args, properties);
  NEED(args->executable, "executable");
  auto& e = exe_of(args->executable);
  args->properties = e.cost_properties.data();
  args->num_properties = e.cost_properties.size();
  return nullptr;
}
PJRT_Error* Executable_OutputMemoryKinds(PJRT_Executable_OutputMemoryKinds_Args* args) {
  NEED_ARGS(PJRT_Executable_OutputMemoryKinds_Args, memory_kind_sizes);
  NEED(args->executable, "executable");
  auto& e = exe_of(args->executable);
  args->num_outputs = e.output_types.size();
  args->memory_kinds = e.output_memory_kinds.data();
  args->memory_kind_sizes = e.output_memory_kind_sizes.data();
  return nullptr;
}
PJRT_Error* Executable_OptimizedProgram(PJRT_Executable_OptimizedProgram_Args* args) {
  NEED_ARGS(PJRT_Executable_OptimizedProgram_Args, program);
  NEED(args->executable, "executable");
  NEED(args->program, "program");
  auto& e = exe_of(args->executable);
  PJRT_Program* p = args->program;
  static const char kFormat[] = "mlir";
  p->format = kFormat;
  p->format_size = 4;
  if (!p->code) {
    p->code_size = e.program_text.size();
    return nullptr;
  }
  if (p->code_size < e.program_text.size())
    return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, "program buffer is too small");
  memcpy(p->code, e.program_text.data(), e.program_text.size());
  p->code_size = e.program_text.size();
  return nullptr;
}
PJRT_Error* Executable_Fingerprint(PJRT_Executable_Fingerprint_Args* args) {
  NEED_ARGS(PJRT_Executable_Fingerprint_Args, executable_fingerprint_size);
  NEED(args->executable, "executable");
  auto& e = exe_of(args->executable);
  args->executable_fingerprint = e.fingerprint.c_str();
  args->executable_fingerprint_size = e.fingerprint.size();
  return nullptr;
}
PJRT_Error* Executable_OutputElementTypes(PJRT_Executable_OutputElementTypes_Args* args) {
  NEED_ARGS(PJRT_Executable_OutputElementTypes_Args, num_output_types);
  NEED(args->executable, "executable");
  auto& e = exe_of(args->executable);
  args->output_types = e.output_types.data();
  args->num_output_types = e.output_types.size();
  return nullptr;
}
PJRT_Error* Executable_OutputDimensions(PJRT_Executable_OutputDimensions_Args* args) {
  NEED_ARGS(PJRT_Executable_OutputDimensions_Args, dim_sizes);
  NEED(args->executable, "executable");
  auto& e = exe_of(args->executable);
  args->num_outputs = e.output_types.size();
  args->dims = e.output_dims_flat.data();
  args->dim_sizes = e.output_ranks.data();
  return nullptr;
}
PJRT_Error* Executable_GetCompileOptions(PJRT_Executable_GetCompileOptions_Args* args) {
  NEED_ARGS(PJRT_Executable_GetCompileOptions_Args, serialized_compile_options_deleter);
  NEED(args->executable, "executable");
  auto& e = exe_of(const_cast<PJRT_Executable*>(args->executable));
  auto* copy = new std::string(e.compile_options);
  args->serialized_bytes = copy->data();
  args->serialized_bytes_size = copy->size();
  args->serialized_compile_options = reinterpret_cast<PJRT_SerializedCompileOptions*>(copy);
  args->serialized_compile_options_deleter = [](PJRT_SerializedCompileOptions* p) {
    delete reinterpret_cast<std::string*>(p);
  };
  return nullptr;
}

PJRT_Error* Executable_Serialize(PJRT_Executable_Serialize_Args* args) {
  NEED_ARGS(PJRT_Executable_Serialize_Args, serialized_executable_deleter);
  NEED(args->executable, "executable");
  API_TRY
  auto& e = exe_of(const_cast<PJRT_Executable*>(args->executable));
  auto* blob = new std::string(serialize_executable(e));
  args->serialized_bytes = blob->data();
  args->serialized_bytes_size = blob->size();
  args->serialized_executable = reinterpret_cast<PJRT_SerializedExecutable*>(blob);
  args->serialized_executable_deleter = [](PJRT_SerializedExecutable* p) { delete reinterpret_cast<std::string*>(p); };
  API_CATCH
}
PJRT_Error* Executable_DeserializeAndLoad(PJRT_Executable_DeserializeAndLoad_Args* args) {
  NEED_ARGS(PJRT_Executable_DeserializeAndLoad_Args, loaded_executable);
  NEED(args->client, "client");
  API_TRY
  Client* c = from<Client>(args->client);
  std::string override_opts;
  const std::string* opts = nullptr;
  const bool has_override =
      args->struct_size >= offsetof(PJRT_Executable_DeserializeAndLoad_Args, overridden_serialized_compile_options_size) +
                               sizeof(size_t) &&
      args->overridden_serialized_compile_options && args->overridden_serialized_compile_options_size > 0;
  if (has_override) {
    override_opts.assign(args->overridden_serialized_compile_options, args->overridden_serialized_compile_options_size);
    opts = &override_opts;
  }
  auto exe = deserialize_executable(c, args->serialized_executable, args->serialized_executable_size, opts);
  args->loaded_executable = to<PJRT_LoadedExecutable>(load_executable(c, std::move(exe)));
  API_CATCH
}
PJRT_Error* Executable_GetCompiledMemoryStats(PJRT_Executable_GetCompiledMemoryStats_Args* args) {
  NEED_ARGS(PJRT_Executable_GetCompiledMemoryStats_Args, peak_memory_in_bytes);
  NEED(args->executable, "executable");
  auto& e = exe_of(args->executable);
  int64_t arg = 0, out = 0, temp = 0, cst = 0;
  for (const Slot& sl : e.plan.slots) {
    const int64_t n = (int64_t)sl.type.bytes();
    if (sl.kind == Slot::PARAM) arg += n;
    else if (sl.kind == Slot::OUTPUT) out += n;
    else if (sl.kind == Slot::TEMP) temp += n;
    else cst += n;
  }
  int64_t alias = 0;  // results that can take over a donated argument's memory
  for (size_t o = 0; o < e.plan.output_alias.size(); ++o)
    if (e.plan.output_alias[o] >= 0) alias += (int64_t)e.plan.output_types[o].bytes();
  // kernels are compiled into the plugin; the executable's device memory is its arguments, outputs, planned
  // temporaries and uploaded constants
  args->generated_code_size_in_bytes = 0;
  args->argument_size_in_bytes = arg;
  args->output_size_in_bytes = out;
  args->alias_size_in_bytes = alias;
  args->temp_size_in_bytes = temp;
  args->host_generated_code_size_in_bytes = 0;
  args->host_argument_size_in_bytes = 0;
  args->host_output_size_in_bytes = 0;
  args->host_alias_size_in_bytes = 0;
  args->host_temp_size_in_bytes = 0;
  args->peak_memory_in_bytes = arg + out + temp + cst;
  auto fits = [&](size_t off) { return args->struct_size >= off + sizeof(int64_t); };
  if (fits(offsetof(PJRT_Executable_GetCompiledMemoryStats_Args, total_size_in_bytes)))
    args->total_size_in_bytes = arg + out + temp + cst;
  if (fits(offsetof(PJRT_Executable_GetCompiledMemoryStats_Args, total_allocation_bytes)))
    args->total_allocation_bytes = out + temp + cst;
  if (fits(offsetof(PJRT_Executable_GetCompiledMemoryStats_Args, indefinite_allocations)))
    args->indefinite_allocations = 0;
  if (fits(offsetof(PJRT_Executable_GetCompiledMemoryStats_Args, peak_unpadded_heap_bytes)))
    args->peak_unpadded_heap_bytes = arg + out + temp + cst;
  return nullptr;
}
PJRT_Error* Executable_ParameterMemoryKinds(PJRT_Executable_ParameterMemoryKinds_Args* args) {
  NEED_ARGS(PJRT_Executable_ParameterMemoryKinds_Args, memory_kind_sizes);
  NEED(args->executable, "executable");
  auto& e = exe_of(args->executable);
  args->num_parameters = e.param_memory_kinds.size();
  args->memory_kinds = e.param_memory_kinds.data();
  args->memory_kind_sizes = e.param_memory_kind_sizes.data();
  return nullptr;
}
PJRT_Error* ExecuteContext_Create(PJRT_ExecuteContext_Create_Args* args) {
  NEED_ARGS(PJRT_ExecuteContext_Create_Args, context);
  args->context = to<PJRT_ExecuteContext>(new ExecuteContext());
  return nullptr;
}
PJRT_Error* ExecuteContext_Destroy(PJRT_ExecuteContext_Destroy_Args* args) {
  NEED_ARGS(PJRT_ExecuteContext_Destroy_Args, context);
  delete from<ExecuteContext>(args->context);
  return nullptr;
}

PJRT_Error* LoadedExecutable_Destroy(PJRT_LoadedExecutable_Destroy_Args* args) {
  NEED_ARGS(PJRT_LoadedExecutable_Destroy_Args, executable);
  delete from<LoadedExecutable>(args->executable);
  return nullptr;
}
PJRT_Error* LoadedExecutable_GetExecutable(PJRT_LoadedExecutable_GetExecutable_Args* args) {
  NEED_ARGS(PJRT_LoadedExecutable_GetExecutable_Args, executable);
  NEED(args->loaded_executable, "loaded_executable");
  args->executable = to<PJRT_Executable>(new ExecutableView{from<LoadedExecutable>(args->loaded_executable)->exe});
  return nullptr;
}
PJRT_Error* LoadedExecutable_AddressableDevices(PJRT_LoadedExecutable_AddressableDevices_Args* args) {
  NEED_ARGS(PJRT_LoadedExecutable_AddressableDevices_Args, num_addressable_devices);
  NEED(args->executable, "executable");
  auto* le = from<LoadedExecutable>(args->executable);
  args->addressable_devices = reinterpret_cast<PJRT_Device* const*>(le->devices.data());
  args->num_addressable_devices = le->devices.size();
  return nullptr;
}
PJRT_Error* LoadedExecutable_AddressableDeviceLogicalIds(PJRT_LoadedExecutable_AddressableDeviceLogicalIds_Args* args) {
  NEED_ARGS(PJRT_LoadedExecutable_AddressableDeviceLogicalIds_Args, num_addressable_device_logical_ids);
  NEED(args->executable, "executable");
  auto* le = from<LoadedExecutable>(args->executable);
  args->addressable_device_logical_ids = le->logical_ids.data();
  args->num_addressable_device_logical_ids = le->logical_ids.size();
  return nullptr;
}
// A serialized xla.DeviceAssignmentProto: replica_count = 1 (field 1), computation_count = 1 (field 2), one
// computation_devices entry (field 3) whose packed replica_device_ids (field 1) hold the executable's device id.
PJRT_Error* LoadedExecutable_GetDeviceAssignment(PJRT_LoadedExecutable_GetDeviceAssignment_Args* args) {
  NEED_ARGS(PJRT_LoadedExecutable_GetDeviceAssignment_Args, serialized_device_assignment_deleter);
  NEED(args->executable, "executable");
  auto* le = from<LoadedExecutable>(args->executable);
  if (le->devices.empty())
    return make_pjrt_error(PJRT_Error_Code_FAILED_PRECONDITION, "a compile-only client has no device assignment");
  auto varint = [](std::string& o, uint64_t v) {
    do {
      uint8_t byte = v & 0x7f;
      v >>= 7;
      o.push_back((char)(byte | (v ? 0x80 : 0)));
    } while (v);
  };
  std::string ids;
  varint(ids, (uint64_t)(int64_t)le->devices[0]->id);
  std::string comp;
  comp.push_back(0x0a);  // replica_device_ids, packed
  varint(comp, ids.size());
  comp += ids;
  auto* blob = new std::string();
  blob->push_back(0x08);  // replica_count
  varint(*blob, 1);
  blob->push_back(0x10);  // computation_count
  varint(*blob, 1);
  blob->push_back(0x1a);  // computation_devices
  varint(*blob, comp.size());
  *blob += comp;
  args->serialized_bytes = blob->data();
  args->serialized_bytes_size = blob->size();
  args->serialized_device_assignment = reinterpret_cast<PJRT_DeviceAssignmentSerialized*>(blob);
  args->serialized_device_assignment_deleter = [](PJRT_DeviceAssignmentSerialized* p) {
    delete reinterpret_cast<std::string*>(p);
  };
  return nullptr;
}
PJRT_Error* LoadedExecutable_Delete(PJRT_LoadedExecutable_Delete_Args* args) {
  NEED_ARGS(PJRT_LoadedExecutable_Delete_Args, executable);
  NEED(args->executable, "executable");
  from<LoadedExecutable>(args->executable)->deleted = true;
  return nullptr;
}
PJRT_Error* LoadedExecutable_IsDeleted(PJRT_LoadedExecutable_IsDeleted_Args* args) {
  NEED_ARGS(PJRT_LoadedExecutable_IsDeleted_Args, is_deleted);
  NEED(args->executable, "executable");
  args->is_deleted = from<LoadedExecutable>(args->executable)->deleted;
  return nullptr;
}
PJRT_Error* LoadedExecutable_Fingerprint(PJRT_LoadedExecutable_Fingerprint_Args* args) {
  NEED_ARGS(PJRT_LoadedExecutable_Fingerprint_Args, executable_fingerprint_size);
  NEED(args->executable, "executable");
  auto* le = from<LoadedExecutable>(args->executable);
  args->executable_fingerprint = le->exe->fingerprint.c_str();
  args->executable_fingerprint_size = le->exe->fingerprint.size();
  return nullptr;
}
PJRT_Error* LoadedExecutable_Execute(PJRT_LoadedExecutable_Execute_Args* args) {
  NEED_ARGS(PJRT_LoadedExecutable_Execute_Args, execute_device);
  NEED(args->executable, "executable");
  API_TRY
  auto* le = from<LoadedExecutable>(args->executable);
  if (le->deleted) return make_pjrt_error(PJRT_Error_Code_FAILED_PRECONDITION, "executable has been deleted");
  if (args->options && args->options->num_send_ops + args->options->num_recv_ops > 0)
    return make_pjrt_error(PJRT_Error_Code_UNIMPLEMENTED, "host send/recv callbacks are not supported");
  size_t nd = args->num_devices;
  if (args->execute_device) {
    if (nd != 1) return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, "execute_device requires exactly one argument list");
    // constants and plans live on the executable's devices only
    Device* want = from<Device>(args->execute_device);
    if (std::find(le->devices.begin(), le->devices.end(), want) == le->devices.end())
      return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, "execute_device is not a device of this executable");
  } else if (nd != le->devices.size()) {
    return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT,
                           "expected argument lists for " + std::to_string(le->devices.size()) + " device(s) but got " +
                               std::to_string(nd));
  }
  // outputs are created by the execution: without somewhere to put them they could never be destroyed
  if (!args->output_lists) return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, "output_lists is null");
  for (size_t d = 0; d < nd; ++d)
    if (!args->output_lists[d]) return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, "output list is null");
  for (size_t d = 0; d < nd; ++d) {
    Device* dev = args->execute_device ? from<Device>(args->execute_device) : le->devices[d];
    std::vector<Buffer*> outs;
    Buffer* const* argv = reinterpret_cast<Buffer* const*>(args->argument_lists ? args->argument_lists[d] : nullptr);
    if (!argv && args->num_args) return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, "argument list is null");
    const PJRT_ExecuteOptions* o = args->options;
    EventPtr done = execute(le, dev, argv, args->num_args, &outs, o ? o->non_donatable_input_indices : nullptr,
                            o ? o->num_non_donatable_input_indices : 0, o ? o->launch_id : 0);
    for (size_t o = 0; o < outs.size(); ++o) args->output_lists[d][o] = to<PJRT_Buffer>(outs[o]);
    if (args->device_complete_events) args->device_complete_events[d] = wrap_event(done);
  }
  API_CATCH
}

// ------------------------------------------------------------------------------------------------ buffers
Buffer* buf(PJRT_Buffer* b) { return from<Buffer>(b); }

PJRT_Error* Buffer_Destroy(PJRT_Buffer_Destroy_Args* args) {
  NEED_ARGS(PJRT_Buffer_Destroy_Args, buffer);
  delete buf(args->buffer);
  return nullptr;
}
PJRT_Error* Buffer_ElementType(PJRT_Buffer_ElementType_Args* args) {
  NEED_ARGS(PJRT_Buffer_ElementType_Args, type);
  NEED(args->buffer, "buffer");
  args->type = (PJRT_Buffer_Type)buf(args->buffer)->dtype;
  return nullptr;
}
PJRT_Error* Buffer_Dimensions(PJRT_Buffer_Dimensions_Args* args) {
  NEED_ARGS(PJRT_Buffer_Dimensions_Args, num_dims);
  NEED(args->buffer, "buffer");
  Buffer* b = buf(args->buffer);
  args->dims = b->dims.data();
  args->num_dims = b->dims.size();
  return nullptr;
}
PJRT_Error* Buffer_UnpaddedDimensions(PJRT_Buffer_UnpaddedDimensions_Args* args) {
  NEED_ARGS(PJRT_Buffer_UnpaddedDimensions_Args, num_dims);
  NEED(args->buffer, "buffer");
  Buffer* b = buf(args->buffer);
  args->unpadded_dims = b->dims.data();
  args->num_dims = b->dims.size();
  return nullptr;
}
PJRT_Error* Buffer_DynamicDimensionIndices(PJRT_Buffer_DynamicDimensionIndices_Args* args) {
  NEED_ARGS(PJRT_Buffer_DynamicDimensionIndices_Args, num_dynamic_dims);
  args->dynamic_dim_indices = nullptr;
  args->num_dynamic_dims = 0;
  return nullptr;
}
PJRT_Error* Buffer_GetMemoryLayout(PJRT_Buffer_GetMemoryLayout_Args* args) {
  NEED_ARGS(PJRT_Buffer_GetMemoryLayout_Args, layout);
  NEED(args->buffer, "buffer");
  Buffer* b = buf(args->buffer);
  memset(&args->layout, 0, sizeof(args->layout));
  args->layout.struct_size = sizeof(PJRT_Buffer_MemoryLayout);
  args->layout.type = PJRT_Buffer_MemoryLayout_Type_Tiled;
  args->layout.tiled.struct_size = sizeof(PJRT_Buffer_MemoryLayout_Tiled);
  args->layout.tiled.minor_to_major = b->minor_to_major.data();
  args->layout.tiled.minor_to_major_size = b->minor_to_major.size();
  args->layout.tiled.num_tiles = 0;
  return nullptr;
}
PJRT_Error* Buffer_OnDeviceSizeInBytes(PJRT_Buffer_OnDeviceSizeInBytes_Args* args) {
  NEED_ARGS(PJRT_Buffer_OnDeviceSizeInBytes_Args, on_device_size_in_bytes);
  NEED(args->buffer, "buffer");
  args->on_device_size_in_bytes = buf(args->buffer)->bytes();
  return nullptr;
}
PJRT_Error* Buffer_Device(PJRT_Buffer_Device_Args* args) {
  NEED_ARGS(PJRT_Buffer_Device_Args, device);
  NEED(args->buffer, "buffer");
  args->device = to<PJRT_Device>(buf(args->buffer)->device);
  return nullptr;
}
PJRT_Error* Buffer_Memory(PJRT_Buffer_Memory_Args* args) {
  NEED_ARGS(PJRT_Buffer_Memory_Args, memory);
  NEED(args->buffer, "buffer");
  args->memory = to<PJRT_Memory>(buf(args->buffer)->device->default_memory);
  return nullptr;
}
PJRT_Error* Buffer_Delete(PJRT_Buffer_Delete_Args* args) {
  NEED_ARGS(PJRT_Buffer_Delete_Args, buffer);
  NEED(args->buffer, "buffer");
  Buffer* b = buf(args->buffer);
  b->deleted = true;
  b->mem.reset();
  return nullptr;
}
PJRT_Error* Buffer_IsDeleted(PJRT_Buffer_IsDeleted_Args* args) {
  NEED_ARGS(PJRT_Buffer_IsDeleted_Args, is_deleted);
  NEED(args->buffer, "buffer");
  args->is_deleted = buf(args->buffer)->deleted;
  return nullptr;
}
PJRT_Error* Buffer_CopyToDevice(PJRT_Buffer_CopyToDevice_Args* args) {
  NEED_ARGS(PJRT_Buffer_CopyToDevice_Args, dst_buffer);
  NEED(args->buffer, "buffer");
  NEED(args->dst_device, "dst_device");
  API_TRY
  args->dst_buffer = to<PJRT_Buffer>(copy_buffer(buf(args->buffer), from<Device>(args->dst_device)));
  API_CATCH
}
PJRT_Error* Buffer_CopyToMemory(PJRT_Buffer_CopyToMemory_Args* args) {
  NEED_ARGS(PJRT_Buffer_CopyToMemory_Args, dst_buffer);
  NEED(args->buffer, "buffer");
  NEED(args->dst_memory, "dst_memory");
  API_TRY
  args->dst_buffer = to<PJRT_Buffer>(copy_buffer(buf(args->buffer), from<Memory>(args->dst_memory)->devices.at(0)));
  API_CATCH
}
PJRT_Error* Buffer_ToHostBuffer(PJRT_Buffer_ToHostBuffer_Args* args) {
  NEED_ARGS(PJRT_Buffer_ToHostBuffer_Args, event);
  NEED(args->src, "src");
  API_TRY
  Buffer* b = buf(args->src);
  if (args->host_layout) {
    const PJRT_Buffer_MemoryLayout* l = args->host_layout;
    bool dense = l->type == PJRT_Buffer_MemoryLayout_Type_Tiled && l->tiled.num_tiles == 0;
    if (dense && l->tiled.minor_to_major) {
      for (size_t i = 0; i < l->tiled.minor_to_major_size; ++i)
        if (l->tiled.minor_to_major[i] != (int64_t)(l->tiled.minor_to_major_size - 1 - i)) dense = false;
    }
    if (!dense) return make_pjrt_error(PJRT_Error_Code_UNIMPLEMENTED, "only the dense row-major host layout is supported");
  }
  if (!args->dst) {
    args->dst_size = b->bytes();
    return nullptr;
  }
  args->event = wrap_event(buffer_to_host(b, args->dst, args->dst_size));
  API_CATCH
}
PJRT_Error* Buffer_CopyRawToHost(PJRT_Buffer_CopyRawToHost_Args* args) {
  NEED_ARGS(PJRT_Buffer_CopyRawToHost_Args, event);
  NEED(args->buffer, "buffer");
  API_TRY
  args->event = wrap_event(buffer_raw_to_host(buf(args->buffer), args->dst, args->offset, args->transfer_size));
  API_CATCH
}
PJRT_Error* Buffer_IsOnCpu(PJRT_Buffer_IsOnCpu_Args* args) {
  NEED_ARGS(PJRT_Buffer_IsOnCpu_Args, is_on_cpu);
  args->is_on_cpu = false;
  return nullptr;
}
PJRT_Error* Buffer_ReadyEvent(PJRT_Buffer_ReadyEvent_Args* args) {
  NEED_ARGS(PJRT_Buffer_ReadyEvent_Args, event);
  NEED(args->buffer, "buffer");
  args->event = wrap_event(buf(args->buffer)->ready);
  return nullptr;
}
PJRT_Error* Buffer_UnsafePointer(PJRT_Buffer_UnsafePointer_Args* args) {
  NEED_ARGS(PJRT_Buffer_UnsafePointer_Args, buffer_pointer);
  NEED(args->buffer, "buffer");
  Buffer* b = buf(args->buffer);
  args->buffer_pointer = b->mem ? (uintptr_t)b->mem->ptr : 0;
  return nullptr;
}
PJRT_Error* Buffer_IncreaseExternalReferenceCount(PJRT_Buffer_IncreaseExternalReferenceCount_Args* args) {
  NEED_ARGS(PJRT_Buffer_IncreaseExternalReferenceCount_Args, buffer);
  NEED(args->buffer, "buffer");
  buf(args->buffer)->external_refs++;
  return nullptr;
}
PJRT_Error* Buffer_DecreaseExternalReferenceCount(PJRT_Buffer_DecreaseExternalReferenceCount_Args* args) {
  NEED_ARGS(PJRT_Buffer_DecreaseExternalReferenceCount_Args, buffer);
  NEED(args->buffer, "buffer");
  Buffer* b = buf(args->buffer);
  if (b->external_refs.load() <= 0)
    return make_pjrt_error(PJRT_Error_Code_FAILED_PRECONDITION, "external reference count is already zero");
  b->external_refs--;
  return nullptr;
}
PJRT_Error* Buffer_OpaqueDeviceMemoryDataPointer(PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args* args) {
  NEED_ARGS(PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args, device_memory_ptr);
  NEED(args->buffer, "buffer");
  Buffer* b = buf(args->buffer);
  args->device_memory_ptr = b->mem ? b->mem->ptr : nullptr;
  return nullptr;
}

// ------------------------------------------------------------------------------------------------ extension
PJRT_Error* Ext_SetKernelTiming(PJRT_Client* client, bool enable) {
  if (!client) return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, "client is null");
  Client* c = from<Client>(client);
  std::lock_guard<std::mutex> lk(c->prof_mu);
  c->profiling = enable;
  return nullptr;
}
PJRT_Error* Ext_KernelTiming(PJRT_Client* client, const char** json, size_t* size) {
  if (!client || !json || !size) return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, "null argument");
  API_TRY
  static thread_local std::string out;
  out = kernel_timing_json(from<Client>(client));
  *json = out.c_str();
  *size = out.size();
  API_CATCH
}
PJRT_Error* Ext_DescribePlan(PJRT_LoadedExecutable* executable, const char** text, size_t* size) {
  if (!executable || !text || !size) return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, "null argument");
  API_TRY
  auto* le = from<LoadedExecutable>(executable);
  static thread_local std::string out;
  out = le->exe->plan.describe();
  *text = out.c_str();
  *size = out.size();
  API_CATCH
}

// ------------------------------------------------------------------------------------------------ layouts extension
// Buffers are dense and row-major: every layout is {rank-1, ..., 0} with no tiles, written as XLA prints a layout.
PJRT_Error* Layouts_MemoryLayout_Destroy(PJRT_Layouts_MemoryLayout_Destroy_Args* args) {
  NEED_ARGS(PJRT_Layouts_MemoryLayout_Destroy_Args, layout);
  delete from<MemoryLayout>(args->layout);
  return nullptr;
}
PJRT_Error* Layouts_MemoryLayout_Serialize(PJRT_Layouts_MemoryLayout_Serialize_Args* args) {
  NEED_ARGS(PJRT_Layouts_MemoryLayout_Serialize_Args, serialized_layout_deleter);
  NEED(args->layout, "layout");
  const MemoryLayout* l = from<MemoryLayout>(args->layout);
  auto* text = new std::string("{");
  for (size_t i = 0; i < l->minor_to_major.size(); ++i) *text += (i ? "," : "") + std::to_string(l->minor_to_major[i]);
  *text += "}";
  args->serialized_bytes = text->data();
  args->serialized_bytes_size = text->size();
  args->serialized_layout = reinterpret_cast<PJRT_Layouts_SerializedLayout*>(text);
  args->serialized_layout_deleter = [](PJRT_Layouts_SerializedLayout* p) { delete reinterpret_cast<std::string*>(p); };
  return nullptr;
}
PJRT_Error* Layouts_Client_GetDefaultLayout(PJRT_Layouts_PJRT_Client_GetDefaultLayout_Args* args) {
  NEED_ARGS(PJRT_Layouts_PJRT_Client_GetDefaultLayout_Args, layout);
  NEED(args->client, "client");
  if (args->num_dims && !args->dims) return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, "dims is null");
  for (size_t i = 0; i < args->num_dims; ++i)
    if (args->dims[i] < 0) return make_pjrt_error(PJRT_Error_Code_INVALID_ARGUMENT, "negative dimension");
  auto* l = new MemoryLayout();
  for (size_t i = 0; i < args->num_dims; ++i) l->minor_to_major.push_back((int64_t)(args->num_dims - 1 - i));
  args->layout = to<PJRT_Layouts_MemoryLayout>(l);
  return nullptr;
}
PJRT_Error* Layouts_Buffer_MemoryLayout(PJRT_Layouts_PJRT_Buffer_MemoryLayout_Args* args) {
  NEED_ARGS(PJRT_Layouts_PJRT_Buffer_MemoryLayout_Args, layout);
  NEED(args->buffer, "buffer");
  auto* l = new MemoryLayout();
  l->minor_to_major = buf(args->buffer)->minor_to_major;
  args->layout = to<PJRT_Layouts_MemoryLayout>(l);
  return nullptr;
}
PJRT_Error* Layouts_Executable_GetOutputLayouts(PJRT_Layouts_PJRT_Executable_GetOutputLayouts_Args* args) {
  NEED_ARGS(PJRT_Layouts_PJRT_Executable_GetOutputLayouts_Args, layouts);
  NEED(args->executable, "executable");
  auto& e = exe_of(args->executable);
  args->num_outputs = e.output_layout_ptrs.size();
  args->layouts = reinterpret_cast<PJRT_Layouts_MemoryLayout**>(e.output_layout_ptrs.data());
  return nullptr;
}
PJRT_Error* Layouts_Executable_GetParameterLayouts(PJRT_Layouts_PJRT_Executable_GetParameterLayouts_Args* args) {
  NEED_ARGS(PJRT_Layouts_PJRT_Executable_GetParameterLayouts_Args, layouts);
  NEED(args->executable, "executable");
  auto& e = exe_of(args->executable);
  args->num_parameters = e.param_layout_ptrs.size();
  args->layouts = reinterpret_cast<PJRT_Layouts_MemoryLayout**>(e.param_layout_ptrs.data());
  return nullptr;
}

// ------------------------------------------------------------------------------------------------ memory descriptions
// Every device has one memory, HBM, of kind "device"; it is the default.
struct MemoryDescriptionObj {
  const char* kind;
  int kind_id;
};
const MemoryDescriptionObj g_device_memory_description = {"device", kDeviceMemoryKindId};
const MemoryDescriptionObj* const g_memory_descriptions[1] = {&g_device_memory_description};

PJRT_Error* MemDesc_DeviceDescription_MemoryDescriptions(PJRT_DeviceDescription_MemoryDescriptions_Args* args) {
  NEED_ARGS(PJRT_DeviceDescription_MemoryDescriptions_Args, default_memory_index);
  NEED(args->device_description, "device_description");
  args->memory_descriptions = reinterpret_cast<const PJRT_MemoryDescription* const*>(g_memory_descriptions);
  args->num_memory_descriptions = 1;
  args->default_memory_index = 0;
  return nullptr;
}
PJRT_Error* MemDesc_MemoryDescription_Kind(PJRT_MemoryDescription_Kind_Args* args) {
  NEED_ARGS(PJRT_MemoryDescription_Kind_Args, kind_id);
  NEED(args->memory_description, "memory_description");
  auto* d = reinterpret_cast<const MemoryDescriptionObj*>(args->memory_description);
  args->kind = d->kind;
  args->kind_size = strlen(d->kind);
  args->kind_id = d->kind_id;
  return nullptr;
}

PJRT_MemoryDescriptions_Extension g_memory_descriptions_extension = {
    {sizeof(PJRT_MemoryDescriptions_Extension), PJRT_Extension_Type_MemoryDescriptions, &g_profiler_extension.base},
    MemDesc_DeviceDescription_MemoryDescriptions,
    MemDesc_MemoryDescription_Kind,
};

PJRT_Layouts_Extension g_layouts_extension = {
    {sizeof(PJRT_Layouts_Extension), PJRT_Extension_Type_Layouts, &g_memory_descriptions_extension.base},
    Layouts_MemoryLayout_Destroy,
    Layouts_MemoryLayout_Serialize,
    Layouts_Client_GetDefaultLayout,
    Layouts_Buffer_MemoryLayout,
    nullptr,
    Layouts_Executable_GetOutputLayouts,
    Layouts_Executable_GetParameterLayouts,
};

RYFT_MI355X_Extension g_extension = {
    {sizeof(RYFT_MI355X_Extension), (PJRT_Extension_Type)RYFT_MI355X_EXTENSION_TYPE, &g_layouts_extension.base},
    Ext_SetKernelTiming,
    Ext_KernelTiming,
    Ext_DescribePlan,
};

PJRT_Api make_api() {
  PJRT_Api a;
  memset(&a, 0, sizeof(a));
  a.struct_size = sizeof(PJRT_Api);
  a.extension_start = &g_extension.base;
  a.pjrt_api_version.struct_size = sizeof(PJRT_Api_Version);
  a.pjrt_api_version.major_version = PJRT_API_MAJOR;
  a.pjrt_api_version.minor_version = PJRT_API_MINOR;
#define SET(name) a.PJRT_##name = name
  SET(Error_Destroy);
  SET(Error_Message);
  SET(Error_GetCode);
  SET(Error_ForEachPayload);
  SET(Plugin_Initialize);
  SET(Plugin_Attributes);
  SET(Event_Destroy);
  SET(Event_IsReady);
  SET(Event_Error);
  SET(Event_Await);
  SET(Event_OnReady);
  SET(Event_Create);
  SET(Event_Set);
  SET(Client_Create);
  SET(Client_Destroy);
  SET(Client_PlatformName);
  SET(Client_ProcessIndex);
  SET(Client_PlatformVersion);
  SET(Client_Devices);
  SET(Client_AddressableDevices);
  SET(Client_LookupDevice);
  SET(Client_LookupAddressableDevice);
  SET(Client_AddressableMemories);
  SET(Client_Compile);
  SET(Client_DefaultDeviceAssignment);
  SET(Client_BufferFromHostBuffer);
  SET(Client_CreateUninitializedBuffer);
  SET(Client_CreateErrorBuffer);
  SET(DeviceDescription_Id);
  SET(DeviceDescription_ProcessIndex);
  SET(DeviceDescription_Attributes);
  SET(DeviceDescription_Kind);
  SET(DeviceDescription_DebugString);
  SET(DeviceDescription_ToString);
  SET(Device_GetDescription);
  SET(Device_IsAddressable);
  SET(Device_LocalHardwareId);
  SET(Device_AddressableMemories);
  SET(Device_DefaultMemory);
  SET(Device_MemoryStats);
  SET(Device_PoisonExecution);
  SET(Memory_Id);
  SET(Memory_Kind);
  SET(Memory_Kind_Id);
  SET(Memory_DebugString);
  SET(Memory_ToString);
  SET(Memory_AddressableByDevices);
  SET(Executable_Destroy);
  SET(Executable_Name);
  SET(Executable_NumReplicas);
  SET(Executable_NumPartitions);
  SET(Executable_NumOutputs);
  SET(Executable_SizeOfGeneratedCodeInBytes);
  SET(Executable_GetCostAnalysis);
  SET(Executable_OutputMemoryKinds);
  SET(Executable_OptimizedProgram);
  SET(Executable_Fingerprint);
  SET(Executable_OutputElementTypes);
  SET(Executable_OutputDimensions);
  SET(Executable_GetCompileOptions);
  SET(Executable_Serialize);
  SET(Executable_DeserializeAndLoad);
  SET(Executable_GetCompiledMemoryStats);
  SET(Executable_ParameterMemoryKinds);
  SET(ExecuteContext_Create);
  SET(ExecuteContext_Destroy);
  SET(LoadedExecutable_GetDeviceAssignment);
  SET(Buffer_CopyRawToHost);
  SET(LoadedExecutable_Destroy);
  SET(LoadedExecutable_GetExecutable);
  SET(LoadedExecutable_AddressableDevices);
  SET(LoadedExecutable_AddressableDeviceLogicalIds);
  SET(LoadedExecutable_Delete);
  SET(LoadedExecutable_IsDeleted);
  SET(LoadedExecutable_Fingerprint);
  SET(LoadedExecutable_Execute);
  SET(Buffer_Destroy);
  SET(Buffer_ElementType);
  SET(Buffer_Dimensions);
  SET(Buffer_UnpaddedDimensions);
  SET(Buffer_DynamicDimensionIndices);
  SET(Buffer_GetMemoryLayout);
  SET(Buffer_OnDeviceSizeInBytes);
  SET(Buffer_Device);
  SET(Buffer_Memory);
  SET(Buffer_Delete);
  SET(Buffer_IsDeleted);
  SET(Buffer_CopyToDevice);
  SET(Buffer_CopyToMemory);
  SET(Buffer_ToHostBuffer);
  SET(Buffer_IsOnCpu);
  SET(Buffer_ReadyEvent);
  SET(Buffer_UnsafePointer);
  SET(Buffer_IncreaseExternalReferenceCount);
  SET(Buffer_DecreaseExternalReferenceCount);
  SET(Buffer_OpaqueDeviceMemoryDataPointer);
#undef SET
  return a;
}

}  // namespace

extern "C" __attribute__((visibility("default"))) const PJRT_Api* GetPjrtApi(void) {
  static const PJRT_Api api = make_api();
  return &api;
}
