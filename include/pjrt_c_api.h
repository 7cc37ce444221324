/*
 * PJRT C API, version 0.104 — the ABI the MI355X plugin exports through GetPjrtApi().
 *
 * This header restates, in C, the `#[repr(C)]` FFI layouts that ryft-pjrt binds. Every struct,
 * enum value and table slot below is laid out exactly as the reference's Rust definitions so a
 * caller compiled against ryft-pjrt sees identical offsets. Sources (reference tree):
 *   PJRT_Api table order ............ crates/ryft-pjrt/src/lib.rs:214-364
 *   PJRT_Extension_Base / types ..... crates/ryft-pjrt/src/lib.rs:166-212
 *   version 0.104 ................... crates/ryft-pjrt/src/versions.rs:30-48
 *   errors .......................... crates/ryft-pjrt/src/errors.rs:404-525
 *   events .......................... crates/ryft-pjrt/src/events.rs:364-560
 *   plugin init / attributes ........ crates/ryft-pjrt/src/plugins.rs:172-210
 *   named values .................... crates/ryft-pjrt/src/values.rs:211-263
 *   clients ......................... crates/ryft-pjrt/src/clients.rs:829-1200
 *   devices / descriptions .......... crates/ryft-pjrt/src/devices.rs:766-1180
 *   memories ........................ crates/ryft-pjrt/src/memories.rs:195-330
 *   programs / executables .......... crates/ryft-pjrt/src/programs.rs:1485-2450
 *   buffers ......................... crates/ryft-pjrt/src/buffers.rs:2549-3400
 *
 * Table slots this plugin does not implement are declared with the opaque PJRT_Unimplemented_Fn type:
 * they are pointer-sized and left null, which ryft-pjrt reports as Error::Unimplemented
 * (crates/ryft-pjrt/src/macros.rs:92-96).
 *
 * Layout is checked with static_assert at the end of the file (x86-64 SysV, LP64).
 */
#ifndef RYFT_MI355X_PJRT_C_API_H_
#define RYFT_MI355X_PJRT_C_API_H_

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PJRT_API_MAJOR 0
#define PJRT_API_MINOR 104

/* ---------------------------------------------------------------- extensions */
typedef unsigned int PJRT_Extension_Type;
enum {
  PJRT_Extension_Type_Gpu_Custom_Call = 0,
  PJRT_Extension_Type_Profiler = 1,
  PJRT_Extension_Type_Custom_Partitioner = 2,
  PJRT_Extension_Type_Stream = 3,
  PJRT_Extension_Type_Layouts = 4,
  PJRT_Extension_Type_FFI = 5,
  PJRT_Extension_Type_MemoryDescriptions = 6,
  PJRT_Extension_Type_Triton = 7,
  PJRT_Extension_Type_RawBuffer = 8,
  PJRT_Extension_Type_PhaseCompile = 9,
  PJRT_Extension_Type_Example = 10,
  PJRT_Extension_Type_Unknown = 11,
  PJRT_Extension_Type_CrossHostTransfers = 12,
  PJRT_Extension_Type_ExecutableMetadata = 13,
  PJRT_Extension_Type_Callback = 14,
  PJRT_Extension_Type_HostAllocator = 15,
  PJRT_Extension_Type_TpuTopology = 16,
  PJRT_Extension_Type_TpuExecutable = 17,
  PJRT_Extension_Type_Megascale = 18,
  PJRT_Extension_Type_Shardings = 19,
  PJRT_Extension_Type_AbiVersion = 20,
  PJRT_Extension_Type_Collectives = 21,
  PJRT_Extension_Type_MultiSlice = 22,
  PJRT_Extension_Type_HostMemoryAllocator = 23,
};

typedef struct PJRT_Extension_Base {
  size_t struct_size;
  PJRT_Extension_Type extension_type;
  struct PJRT_Extension_Base* next;
} PJRT_Extension_Base;

/* Every *_Args struct starts with these two fields. */
#define PJRT_ARGS_HEAD        \
  size_t struct_size;         \
  PJRT_Extension_Base* extension_start

/* ---------------------------------------------------------------- opaque handles */
typedef struct PJRT_Error PJRT_Error;
typedef struct PJRT_Event PJRT_Event;
typedef struct PJRT_Client PJRT_Client;
typedef struct PJRT_Device PJRT_Device;
typedef struct PJRT_DeviceDescription PJRT_DeviceDescription;
typedef struct PJRT_Memory PJRT_Memory;
typedef struct PJRT_Executable PJRT_Executable;
typedef struct PJRT_LoadedExecutable PJRT_LoadedExecutable;
typedef struct PJRT_Buffer PJRT_Buffer;
typedef struct PJRT_TopologyDescription PJRT_TopologyDescription;
typedef struct PJRT_ExecuteContext PJRT_ExecuteContext;
typedef struct PJRT_MultiSlice_Config PJRT_MultiSlice_Config;
typedef struct PJRT_SerializedCompileOptions PJRT_SerializedCompileOptions;
typedef struct PJRT_SerializedExecutable PJRT_SerializedExecutable;
typedef struct PJRT_DeviceAssignmentSerialized PJRT_DeviceAssignmentSerialized;
typedef struct PJRT_Device_Attributes PJRT_Device_Attributes;

typedef void (*PJRT_Unimplemented_Fn)(void);

/* ---------------------------------------------------------------- version (versions.rs:33-48) */
typedef struct PJRT_Api_Version {
  PJRT_ARGS_HEAD;
  int major_version;
  int minor_version;
} PJRT_Api_Version;

/* ---------------------------------------------------------------- errors (errors.rs:404-525) */
typedef unsigned int PJRT_Error_Code;
enum {
  PJRT_Error_Code_OK = 0,
  PJRT_Error_Code_CANCELLED = 1,
  PJRT_Error_Code_UNKNOWN = 2,
  PJRT_Error_Code_INVALID_ARGUMENT = 3,
  PJRT_Error_Code_DEADLINE_EXCEEDED = 4,
  PJRT_Error_Code_NOT_FOUND = 5,
  PJRT_Error_Code_ALREADY_EXISTS = 6,
  PJRT_Error_Code_PERMISSION_DENIED = 7,
  PJRT_Error_Code_RESOURCE_EXHAUSTED = 8,
  PJRT_Error_Code_FAILED_PRECONDITION = 9,
  PJRT_Error_Code_ABORTED = 10,
  PJRT_Error_Code_OUT_OF_RANGE = 11,
  PJRT_Error_Code_UNIMPLEMENTED = 12,
  PJRT_Error_Code_INTERNAL = 13,
  PJRT_Error_Code_UNAVAILABLE = 14,
  PJRT_Error_Code_DATA_LOSS = 15,
  PJRT_Error_Code_UNAUTHENTICATED = 16,
};

typedef struct PJRT_Error_Destroy_Args {
  PJRT_ARGS_HEAD;
  PJRT_Error* error;
} PJRT_Error_Destroy_Args;
typedef void PJRT_Error_Destroy(PJRT_Error_Destroy_Args* args);

typedef struct PJRT_Error_Message_Args {
  PJRT_ARGS_HEAD;
  const PJRT_Error* error;
  const char* message; /* out, borrowed */
  size_t message_size; /* out */
} PJRT_Error_Message_Args;
typedef void PJRT_Error_Message(PJRT_Error_Message_Args* args);

typedef struct PJRT_Error_GetCode_Args {
  PJRT_ARGS_HEAD;
  const PJRT_Error* error;
  PJRT_Error_Code code; /* out */
} PJRT_Error_GetCode_Args;
typedef PJRT_Error* PJRT_Error_GetCode(PJRT_Error_GetCode_Args* args);

typedef void (*PJRT_Error_PayloadVisitor)(const char* key, size_t key_size, const char* value, size_t value_size,
                                          void* user_arg);
typedef struct PJRT_Error_ForEachPayload_Args {
  PJRT_ARGS_HEAD;
  const PJRT_Error* error;
  PJRT_Error_PayloadVisitor visitor;
  void* user_arg;
} PJRT_Error_ForEachPayload_Args;
typedef PJRT_Error* PJRT_Error_ForEachPayload(PJRT_Error_ForEachPayload_Args* args);

typedef PJRT_Error* (*PJRT_CallbackError)(PJRT_Error_Code code, const char* message, size_t message_size);

/* ---------------------------------------------------------------- named values (values.rs:211-263) */
typedef unsigned int PJRT_NamedValue_Type;
enum {
  PJRT_NamedValue_kString = 0,
  PJRT_NamedValue_kInt64 = 1,
  PJRT_NamedValue_kInt64List = 2,
  PJRT_NamedValue_kFloat = 3,
  PJRT_NamedValue_kBool = 4,
};

typedef struct PJRT_NamedValue {
  PJRT_ARGS_HEAD;
  const char* name;
  size_t name_size;
  PJRT_NamedValue_Type type;
  union {
    const char* string_value;
    int64_t int64_value;
    const int64_t* int64_array_value;
    float float_value;
    bool bool_value;
  };
  size_t value_size; /* string length, list length, or 1 */
} PJRT_NamedValue;

/* ---------------------------------------------------------------- plugin (plugins.rs:172-210) */
typedef struct PJRT_Plugin_Initialize_Args {
  PJRT_ARGS_HEAD;
} PJRT_Plugin_Initialize_Args;
typedef PJRT_Error* PJRT_Plugin_Initialize(PJRT_Plugin_Initialize_Args* args);

typedef struct PJRT_Plugin_Attributes_Args {
  PJRT_ARGS_HEAD;
  const PJRT_NamedValue* attributes; /* out, plugin-owned */
  size_t num_attributes;             /* out */
} PJRT_Plugin_Attributes_Args;
typedef PJRT_Error* PJRT_Plugin_Attributes(PJRT_Plugin_Attributes_Args* args);

/* ---------------------------------------------------------------- events (events.rs:364-560) */
typedef struct PJRT_Event_Destroy_Args {
  PJRT_ARGS_HEAD;
  PJRT_Event* event;
} PJRT_Event_Destroy_Args;
typedef PJRT_Error* PJRT_Event_Destroy(PJRT_Event_Destroy_Args* args);

typedef struct PJRT_Event_IsReady_Args {
  PJRT_ARGS_HEAD;
  PJRT_Event* event;
  bool is_ready; /* out */
} PJRT_Event_IsReady_Args;
typedef PJRT_Error* PJRT_Event_IsReady(PJRT_Event_IsReady_Args* args);

typedef struct PJRT_Event_Error_Args {
  PJRT_ARGS_HEAD;
  PJRT_Event* event;
} PJRT_Event_Error_Args;
typedef PJRT_Error* PJRT_Event_Error(PJRT_Event_Error_Args* args);

typedef struct PJRT_Event_Await_Args {
  PJRT_ARGS_HEAD;
  PJRT_Event* event;
} PJRT_Event_Await_Args;
typedef PJRT_Error* PJRT_Event_Await(PJRT_Event_Await_Args* args);

typedef void (*PJRT_Event_OnReadyCallback)(PJRT_Error* error, void* user_arg);
typedef struct PJRT_Event_OnReady_Args {
  PJRT_ARGS_HEAD;
  PJRT_Event* event;
  PJRT_Event_OnReadyCallback callback;
  void* user_arg;
} PJRT_Event_OnReady_Args;
typedef PJRT_Error* PJRT_Event_OnReady(PJRT_Event_OnReady_Args* args);

typedef struct PJRT_Event_Create_Args {
  PJRT_ARGS_HEAD;
  PJRT_Event* event; /* out */
} PJRT_Event_Create_Args;
typedef PJRT_Error* PJRT_Event_Create(PJRT_Event_Create_Args* args);

typedef struct PJRT_Event_Set_Args {
  PJRT_ARGS_HEAD;
  PJRT_Event* event;
  PJRT_Error_Code error_code;
  const char* error_message;
  size_t error_message_size;
} PJRT_Event_Set_Args;
typedef PJRT_Error* PJRT_Event_Set(PJRT_Event_Set_Args* args);

/* ---------------------------------------------------------------- clients (clients.rs:829-1200) */
typedef struct PJRT_KeyValueGetCallback_Args PJRT_KeyValueGetCallback_Args;
typedef struct PJRT_KeyValuePutCallback_Args PJRT_KeyValuePutCallback_Args;
typedef struct PJRT_KeyValueTryGetCallback_Args PJRT_KeyValueTryGetCallback_Args;
typedef PJRT_Error* (*PJRT_KeyValueGetCallback)(PJRT_KeyValueGetCallback_Args* args);
typedef PJRT_Error* (*PJRT_KeyValuePutCallback)(PJRT_KeyValuePutCallback_Args* args);
typedef PJRT_Error* (*PJRT_KeyValueTryGetCallback)(PJRT_KeyValueTryGetCallback_Args* args);

typedef struct PJRT_Client_Create_Args {
  PJRT_ARGS_HEAD;
  const PJRT_NamedValue* create_options;
  size_t num_options;
  PJRT_KeyValueGetCallback kv_get_callback;
  void* kv_get_user_arg;
  PJRT_KeyValuePutCallback kv_put_callback;
  void* kv_put_user_arg;
  PJRT_Client* client; /* out */
  PJRT_KeyValueTryGetCallback kv_try_get_callback;
  void* kv_try_get_user_arg;
} PJRT_Client_Create_Args;
typedef PJRT_Error* PJRT_Client_Create(PJRT_Client_Create_Args* args);

typedef struct PJRT_Client_Destroy_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
} PJRT_Client_Destroy_Args;
typedef PJRT_Error* PJRT_Client_Destroy(PJRT_Client_Destroy_Args* args);

typedef struct PJRT_Client_PlatformName_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  const char* platform_name; /* out */
  size_t platform_name_size; /* out */
} PJRT_Client_PlatformName_Args;
typedef PJRT_Error* PJRT_Client_PlatformName(PJRT_Client_PlatformName_Args* args);

typedef struct PJRT_Client_ProcessIndex_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  int process_index; /* out */
} PJRT_Client_ProcessIndex_Args;
typedef PJRT_Error* PJRT_Client_ProcessIndex(PJRT_Client_ProcessIndex_Args* args);

typedef struct PJRT_Client_PlatformVersion_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  const char* platform_version; /* out */
  size_t platform_version_size; /* out */
} PJRT_Client_PlatformVersion_Args;
typedef PJRT_Error* PJRT_Client_PlatformVersion(PJRT_Client_PlatformVersion_Args* args);

typedef struct PJRT_Client_Devices_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  PJRT_Device* const* devices; /* out */
  size_t num_devices;          /* out */
} PJRT_Client_Devices_Args;
typedef PJRT_Error* PJRT_Client_Devices(PJRT_Client_Devices_Args* args);

typedef struct PJRT_Client_AddressableDevices_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  PJRT_Device* const* addressable_devices; /* out */
  size_t num_addressable_devices;          /* out */
} PJRT_Client_AddressableDevices_Args;
typedef PJRT_Error* PJRT_Client_AddressableDevices(PJRT_Client_AddressableDevices_Args* args);

typedef struct PJRT_Client_LookupDevice_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  int id;
  PJRT_Device* device; /* out */
} PJRT_Client_LookupDevice_Args;
typedef PJRT_Error* PJRT_Client_LookupDevice(PJRT_Client_LookupDevice_Args* args);

typedef struct PJRT_Client_LookupAddressableDevice_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  int local_hardware_id;
  PJRT_Device* addressable_device; /* out */
} PJRT_Client_LookupAddressableDevice_Args;
typedef PJRT_Error* PJRT_Client_LookupAddressableDevice(PJRT_Client_LookupAddressableDevice_Args* args);

typedef struct PJRT_Client_AddressableMemories_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  PJRT_Memory* const* addressable_memories; /* out */
  size_t num_addressable_memories;          /* out */
} PJRT_Client_AddressableMemories_Args;
typedef PJRT_Error* PJRT_Client_AddressableMemories(PJRT_Client_AddressableMemories_Args* args);

typedef struct PJRT_Program {
  PJRT_ARGS_HEAD;
  char* code;
  size_t code_size;
  const char* format; /* "mlir" or "hlo" (programs.rs:56-62) */
  size_t format_size;
} PJRT_Program;

typedef struct PJRT_Client_Compile_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  const PJRT_Program* program;
  const char* compile_options; /* serialized xla.CompileOptionsProto */
  size_t compile_options_size;
  PJRT_LoadedExecutable* executable; /* out */
} PJRT_Client_Compile_Args;
typedef PJRT_Error* PJRT_Client_Compile(PJRT_Client_Compile_Args* args);

typedef struct PJRT_Client_DefaultDeviceAssignment_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  int num_replicas;
  int num_partitions;
  size_t default_assignment_size;
  int* default_assignment; /* caller-owned, filled */
} PJRT_Client_DefaultDeviceAssignment_Args;
typedef PJRT_Error* PJRT_Client_DefaultDeviceAssignment(PJRT_Client_DefaultDeviceAssignment_Args* args);

/* ---------------------------------------------------------------- buffers (buffers.rs:2549-3400) */
typedef unsigned int PJRT_Buffer_Type;
enum {
  PJRT_Buffer_Type_INVALID = 0,
  PJRT_Buffer_Type_PRED = 1,
  PJRT_Buffer_Type_S8 = 2,
  PJRT_Buffer_Type_S16 = 3,
  PJRT_Buffer_Type_S32 = 4,
  PJRT_Buffer_Type_S64 = 5,
  PJRT_Buffer_Type_U8 = 6,
  PJRT_Buffer_Type_U16 = 7,
  PJRT_Buffer_Type_U32 = 8,
  PJRT_Buffer_Type_U64 = 9,
  PJRT_Buffer_Type_F16 = 10,
  PJRT_Buffer_Type_F32 = 11,
  PJRT_Buffer_Type_F64 = 12,
  PJRT_Buffer_Type_BF16 = 13,
  PJRT_Buffer_Type_C64 = 14,
  PJRT_Buffer_Type_C128 = 15,
  PJRT_Buffer_Type_F8E5M2 = 16,
  PJRT_Buffer_Type_F8E4M3FN = 17,
  PJRT_Buffer_Type_F8E4M3B11FNUZ = 18,
  PJRT_Buffer_Type_F8E5M2FNUZ = 19,
  PJRT_Buffer_Type_F8E4M3FNUZ = 20,
  PJRT_Buffer_Type_S4 = 21,
  PJRT_Buffer_Type_U4 = 22,
  PJRT_Buffer_Type_TOKEN = 23,
  PJRT_Buffer_Type_S2 = 24,
  PJRT_Buffer_Type_U2 = 25,
  PJRT_Buffer_Type_F8E4M3 = 26,
  PJRT_Buffer_Type_F8E3M4 = 27,
  PJRT_Buffer_Type_F8E8M0FNU = 28,
  PJRT_Buffer_Type_F4E2M1FN = 29,
  PJRT_Buffer_Type_S1 = 30,
  PJRT_Buffer_Type_U1 = 31,
};

typedef unsigned int PJRT_HostBufferSemantics;
enum {
  PJRT_HostBufferSemantics_kImmutableOnlyDuringCall = 0,
  PJRT_HostBufferSemantics_kImmutableUntilTransferCompletes = 1,
  PJRT_HostBufferSemantics_kImmutableZeroCopy = 2,
  PJRT_HostBufferSemantics_kMutableZeroCopy = 3,
};

typedef unsigned int PJRT_Buffer_MemoryLayout_Type;
enum {
  PJRT_Buffer_MemoryLayout_Type_Tiled = 0,
  PJRT_Buffer_MemoryLayout_Type_Strides = 1,
};

typedef struct PJRT_Buffer_MemoryLayout_Tiled {
  PJRT_ARGS_HEAD;
  const int64_t* minor_to_major;
  size_t minor_to_major_size;
  const int64_t* tile_dims;
  const size_t* tile_dim_sizes;
  size_t num_tiles;
} PJRT_Buffer_MemoryLayout_Tiled;

typedef struct PJRT_Buffer_MemoryLayout_Strides {
  PJRT_ARGS_HEAD;
  const int64_t* byte_strides;
  size_t num_byte_strides;
} PJRT_Buffer_MemoryLayout_Strides;

typedef struct PJRT_Buffer_MemoryLayout {
  PJRT_ARGS_HEAD;
  union {
    PJRT_Buffer_MemoryLayout_Tiled tiled;
    PJRT_Buffer_MemoryLayout_Strides strides;
  };
  PJRT_Buffer_MemoryLayout_Type type;
} PJRT_Buffer_MemoryLayout;

typedef struct PJRT_Client_BufferFromHostBuffer_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  const void* data;
  PJRT_Buffer_Type type;
  const int64_t* dims;
  size_t num_dims;
  const int64_t* byte_strides;
  size_t num_byte_strides;
  PJRT_HostBufferSemantics host_buffer_semantics;
  PJRT_Device* device;
  PJRT_Memory* memory;
  PJRT_Buffer_MemoryLayout* device_layout;
  PJRT_Event* done_with_host_buffer; /* out */
  PJRT_Buffer* buffer;               /* out */
} PJRT_Client_BufferFromHostBuffer_Args;
typedef PJRT_Error* PJRT_Client_BufferFromHostBuffer(PJRT_Client_BufferFromHostBuffer_Args* args);

typedef struct PJRT_Client_CreateUninitializedBuffer_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  const int64_t* shape_dims;
  size_t shape_num_dims;
  PJRT_Buffer_Type shape_element_type;
  PJRT_Buffer_MemoryLayout* shape_layout;
  PJRT_Device* device;
  PJRT_Memory* memory;
  PJRT_Buffer* buffer; /* out */
} PJRT_Client_CreateUninitializedBuffer_Args;
typedef PJRT_Error* PJRT_Client_CreateUninitializedBuffer(PJRT_Client_CreateUninitializedBuffer_Args* args);

/* A buffer that holds an error instead of data (crates/ryft-pjrt/src/buffers.rs:2338-2430, 3415-3430). */
typedef struct PJRT_Client_CreateErrorBuffer_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  PJRT_Error_Code error_code;
  const char* error_message;
  size_t error_message_size;
  const int64_t* shape_dims;
  size_t shape_num_dims;
  PJRT_Buffer_Type shape_element_type;
  PJRT_Buffer_MemoryLayout* shape_layout;
  PJRT_Memory* memory;
  PJRT_Buffer* buffer; /* out */
  const PJRT_NamedValue* payload;
  size_t payload_size;
} PJRT_Client_CreateErrorBuffer_Args;
typedef PJRT_Error* PJRT_Client_CreateErrorBuffer(PJRT_Client_CreateErrorBuffer_Args* args);

typedef struct PJRT_Buffer_Destroy_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
} PJRT_Buffer_Destroy_Args;
typedef PJRT_Error* PJRT_Buffer_Destroy(PJRT_Buffer_Destroy_Args* args);

typedef struct PJRT_Buffer_ElementType_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  PJRT_Buffer_Type type; /* out */
} PJRT_Buffer_ElementType_Args;
typedef PJRT_Error* PJRT_Buffer_ElementType(PJRT_Buffer_ElementType_Args* args);

typedef struct PJRT_Buffer_Dimensions_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  const int64_t* dims; /* out, borrowed */
  size_t num_dims;     /* out */
} PJRT_Buffer_Dimensions_Args;
typedef PJRT_Error* PJRT_Buffer_Dimensions(PJRT_Buffer_Dimensions_Args* args);

typedef struct PJRT_Buffer_UnpaddedDimensions_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  const int64_t* unpadded_dims; /* out */
  size_t num_dims;              /* out */
} PJRT_Buffer_UnpaddedDimensions_Args;
typedef PJRT_Error* PJRT_Buffer_UnpaddedDimensions(PJRT_Buffer_UnpaddedDimensions_Args* args);

typedef struct PJRT_Buffer_DynamicDimensionIndices_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  const size_t* dynamic_dim_indices; /* out */
  size_t num_dynamic_dims;           /* out */
} PJRT_Buffer_DynamicDimensionIndices_Args;
typedef PJRT_Error* PJRT_Buffer_DynamicDimensionIndices(PJRT_Buffer_DynamicDimensionIndices_Args* args);

typedef struct PJRT_Buffer_GetMemoryLayout_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  PJRT_Buffer_MemoryLayout layout; /* out */
} PJRT_Buffer_GetMemoryLayout_Args;
typedef PJRT_Error* PJRT_Buffer_GetMemoryLayout(PJRT_Buffer_GetMemoryLayout_Args* args);

typedef struct PJRT_Buffer_OnDeviceSizeInBytes_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  size_t on_device_size_in_bytes; /* out */
} PJRT_Buffer_OnDeviceSizeInBytes_Args;
typedef PJRT_Error* PJRT_Buffer_OnDeviceSizeInBytes(PJRT_Buffer_OnDeviceSizeInBytes_Args* args);

typedef struct PJRT_Buffer_Device_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  PJRT_Device* device; /* out */
} PJRT_Buffer_Device_Args;
typedef PJRT_Error* PJRT_Buffer_Device(PJRT_Buffer_Device_Args* args);

typedef struct PJRT_Buffer_Memory_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  PJRT_Memory* memory; /* out */
} PJRT_Buffer_Memory_Args;
typedef PJRT_Error* PJRT_Buffer_Memory(PJRT_Buffer_Memory_Args* args);

typedef struct PJRT_Buffer_Delete_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
} PJRT_Buffer_Delete_Args;
typedef PJRT_Error* PJRT_Buffer_Delete(PJRT_Buffer_Delete_Args* args);

typedef struct PJRT_Buffer_IsDeleted_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  bool is_deleted; /* out */
} PJRT_Buffer_IsDeleted_Args;
typedef PJRT_Error* PJRT_Buffer_IsDeleted(PJRT_Buffer_IsDeleted_Args* args);

typedef struct PJRT_Buffer_CopyToDevice_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  PJRT_Device* dst_device;
  PJRT_Buffer* dst_buffer; /* out */
} PJRT_Buffer_CopyToDevice_Args;
typedef PJRT_Error* PJRT_Buffer_CopyToDevice(PJRT_Buffer_CopyToDevice_Args* args);

typedef struct PJRT_Buffer_CopyToMemory_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  PJRT_Memory* dst_memory;
  PJRT_Buffer* dst_buffer; /* out */
} PJRT_Buffer_CopyToMemory_Args;
typedef PJRT_Error* PJRT_Buffer_CopyToMemory(PJRT_Buffer_CopyToMemory_Args* args);

typedef struct PJRT_Buffer_ToHostBuffer_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* src;
  PJRT_Buffer_MemoryLayout* host_layout;
  void* dst;         /* null: only dst_size is written */
  size_t dst_size;   /* in/out */
  PJRT_Event* event; /* out */
} PJRT_Buffer_ToHostBuffer_Args;
typedef PJRT_Error* PJRT_Buffer_ToHostBuffer(PJRT_Buffer_ToHostBuffer_Args* args);

/* Buffer_CopyRawToHost: buffers.rs:2931-2958 (caller: Buffer::copy_raw_to_host_buffer, buffers.rs:1318-1340). Copies
 * transfer_size bytes starting at byte `offset` of the buffer's on-device bytes; the event completes when dst holds them. */
typedef struct PJRT_Buffer_CopyRawToHost_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  void* dst;
  int64_t offset;
  int64_t transfer_size;
  PJRT_Event* event; /* out */
} PJRT_Buffer_CopyRawToHost_Args;
typedef PJRT_Error* PJRT_Buffer_CopyRawToHost(PJRT_Buffer_CopyRawToHost_Args* args);

typedef struct PJRT_Buffer_IsOnCpu_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  bool is_on_cpu; /* out */
} PJRT_Buffer_IsOnCpu_Args;
typedef PJRT_Error* PJRT_Buffer_IsOnCpu(PJRT_Buffer_IsOnCpu_Args* args);

typedef struct PJRT_Buffer_ReadyEvent_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  PJRT_Event* event; /* out */
} PJRT_Buffer_ReadyEvent_Args;
typedef PJRT_Error* PJRT_Buffer_ReadyEvent(PJRT_Buffer_ReadyEvent_Args* args);

typedef struct PJRT_Buffer_UnsafePointer_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  uintptr_t buffer_pointer; /* out */
} PJRT_Buffer_UnsafePointer_Args;
typedef PJRT_Error* PJRT_Buffer_UnsafePointer(PJRT_Buffer_UnsafePointer_Args* args);

typedef struct PJRT_Buffer_IncreaseExternalReferenceCount_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
} PJRT_Buffer_IncreaseExternalReferenceCount_Args;
typedef PJRT_Error* PJRT_Buffer_IncreaseExternalReferenceCount(PJRT_Buffer_IncreaseExternalReferenceCount_Args* args);

typedef struct PJRT_Buffer_DecreaseExternalReferenceCount_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
} PJRT_Buffer_DecreaseExternalReferenceCount_Args;
typedef PJRT_Error* PJRT_Buffer_DecreaseExternalReferenceCount(PJRT_Buffer_DecreaseExternalReferenceCount_Args* args);

typedef struct PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  void* device_memory_ptr; /* out */
} PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args;
typedef PJRT_Error* PJRT_Buffer_OpaqueDeviceMemoryDataPointer(PJRT_Buffer_OpaqueDeviceMemoryDataPointer_Args* args);

/* ---------------------------------------------------------------- devices (devices.rs:766-1180) */
typedef struct PJRT_DeviceDescription_Id_Args {
  PJRT_ARGS_HEAD;
  PJRT_DeviceDescription* device_description;
  int id; /* out */
} PJRT_DeviceDescription_Id_Args;
typedef PJRT_Error* PJRT_DeviceDescription_Id(PJRT_DeviceDescription_Id_Args* args);

typedef struct PJRT_DeviceDescription_ProcessIndex_Args {
  PJRT_ARGS_HEAD;
  PJRT_DeviceDescription* device_description;
  int process_index; /* out */
} PJRT_DeviceDescription_ProcessIndex_Args;
typedef PJRT_Error* PJRT_DeviceDescription_ProcessIndex(PJRT_DeviceDescription_ProcessIndex_Args* args);

typedef struct PJRT_DeviceDescription_Attributes_Args {
  PJRT_ARGS_HEAD;
  PJRT_DeviceDescription* device_description;
  size_t num_attributes;             /* out */
  const PJRT_NamedValue* attributes; /* out */
} PJRT_DeviceDescription_Attributes_Args;
typedef PJRT_Error* PJRT_DeviceDescription_Attributes(PJRT_DeviceDescription_Attributes_Args* args);

typedef struct PJRT_DeviceDescription_Kind_Args {
  PJRT_ARGS_HEAD;
  PJRT_DeviceDescription* device_description;
  const char* device_kind; /* out */
  size_t device_kind_size; /* out */
} PJRT_DeviceDescription_Kind_Args;
typedef PJRT_Error* PJRT_DeviceDescription_Kind(PJRT_DeviceDescription_Kind_Args* args);

typedef struct PJRT_DeviceDescription_DebugString_Args {
  PJRT_ARGS_HEAD;
  PJRT_DeviceDescription* device_description;
  const char* debug_string; /* out */
  size_t debug_string_size; /* out */
} PJRT_DeviceDescription_DebugString_Args;
typedef PJRT_Error* PJRT_DeviceDescription_DebugString(PJRT_DeviceDescription_DebugString_Args* args);

typedef struct PJRT_DeviceDescription_ToString_Args {
  PJRT_ARGS_HEAD;
  PJRT_DeviceDescription* device_description;
  const char* to_string; /* out */
  size_t to_string_size; /* out */
} PJRT_DeviceDescription_ToString_Args;
typedef PJRT_Error* PJRT_DeviceDescription_ToString(PJRT_DeviceDescription_ToString_Args* args);

typedef struct PJRT_Device_GetDescription_Args {
  PJRT_ARGS_HEAD;
  PJRT_Device* device;
  PJRT_DeviceDescription* device_description; /* out */
} PJRT_Device_GetDescription_Args;
typedef PJRT_Error* PJRT_Device_GetDescription(PJRT_Device_GetDescription_Args* args);

typedef struct PJRT_Device_IsAddressable_Args {
  PJRT_ARGS_HEAD;
  PJRT_Device* device;
  bool is_addressable; /* out */
} PJRT_Device_IsAddressable_Args;
typedef PJRT_Error* PJRT_Device_IsAddressable(PJRT_Device_IsAddressable_Args* args);

typedef struct PJRT_Device_LocalHardwareId_Args {
  PJRT_ARGS_HEAD;
  PJRT_Device* device;
  int local_hardware_id; /* out */
} PJRT_Device_LocalHardwareId_Args;
typedef PJRT_Error* PJRT_Device_LocalHardwareId(PJRT_Device_LocalHardwareId_Args* args);

typedef struct PJRT_Device_AddressableMemories_Args {
  PJRT_ARGS_HEAD;
  PJRT_Device* device;
  PJRT_Memory* const* memories; /* out */
  size_t num_memories;          /* out */
} PJRT_Device_AddressableMemories_Args;
typedef PJRT_Error* PJRT_Device_AddressableMemories(PJRT_Device_AddressableMemories_Args* args);

typedef struct PJRT_Device_DefaultMemory_Args {
  PJRT_ARGS_HEAD;
  PJRT_Device* device;
  PJRT_Memory* memory; /* out */
} PJRT_Device_DefaultMemory_Args;
typedef PJRT_Error* PJRT_Device_DefaultMemory(PJRT_Device_DefaultMemory_Args* args);

typedef struct PJRT_Device_MemoryStats_Args {
  PJRT_ARGS_HEAD;
  PJRT_Device* device;
  int64_t bytes_in_use;
  int64_t peak_bytes_in_use;
  bool peak_bytes_in_use_is_set;
  int64_t num_allocs;
  bool num_allocs_is_set;
  int64_t largest_alloc_size;
  bool largest_alloc_size_is_set;
  int64_t bytes_limit;
  bool bytes_limit_is_set;
  int64_t bytes_reserved;
  bool bytes_reserved_is_set;
  int64_t peak_bytes_reserved;
  bool peak_bytes_reserved_is_set;
  int64_t bytes_reservable_limit;
  bool bytes_reservable_limit_is_set;
  int64_t largest_free_block_bytes;
  bool largest_free_block_bytes_is_set;
  int64_t pool_bytes;
  bool pool_bytes_is_set;
  int64_t peak_pool_bytes;
  bool peak_pool_bytes_is_set;
} PJRT_Device_MemoryStats_Args;
typedef PJRT_Error* PJRT_Device_MemoryStats(PJRT_Device_MemoryStats_Args* args);

/* Poisons the earliest unfinished execution with this launch id on the device (crates/ryft-pjrt/src/devices.rs:257-300,
   987-998): its results turn into error buffers carrying the given error. */
typedef struct PJRT_Device_PoisonExecution_Args {
  PJRT_ARGS_HEAD;
  PJRT_Device* device;
  int32_t launch_id;
  PJRT_Error_Code error_code;
  const char* error_message;
  size_t error_message_size;
  bool poisoned; /* out */
  const PJRT_NamedValue* payload;
  size_t payload_size;
} PJRT_Device_PoisonExecution_Args;
typedef PJRT_Error* PJRT_Device_PoisonExecution(PJRT_Device_PoisonExecution_Args* args);

/* ---------------------------------------------------------------- memories (memories.rs:195-330) */
typedef struct PJRT_Memory_Id_Args {
  PJRT_ARGS_HEAD;
  PJRT_Memory* memory;
  int id; /* out */
} PJRT_Memory_Id_Args;
typedef PJRT_Error* PJRT_Memory_Id(PJRT_Memory_Id_Args* args);

typedef struct PJRT_Memory_Kind_Args {
  PJRT_ARGS_HEAD;
  PJRT_Memory* memory;
  const char* kind; /* out */
  size_t kind_size; /* out */
} PJRT_Memory_Kind_Args;
typedef PJRT_Error* PJRT_Memory_Kind(PJRT_Memory_Kind_Args* args);

typedef struct PJRT_Memory_Kind_Id_Args {
  PJRT_ARGS_HEAD;
  PJRT_Memory* memory;
  int kind_id; /* out */
} PJRT_Memory_Kind_Id_Args;
typedef PJRT_Error* PJRT_Memory_Kind_Id(PJRT_Memory_Kind_Id_Args* args);

typedef struct PJRT_Memory_DebugString_Args {
  PJRT_ARGS_HEAD;
  PJRT_Memory* memory;
  const char* debug_string; /* out */
  size_t debug_string_size; /* out */
} PJRT_Memory_DebugString_Args;
typedef PJRT_Error* PJRT_Memory_DebugString(PJRT_Memory_DebugString_Args* args);

typedef struct PJRT_Memory_ToString_Args {
  PJRT_ARGS_HEAD;
  PJRT_Memory* memory;
  const char* to_string; /* out */
  size_t to_string_size; /* out */
} PJRT_Memory_ToString_Args;
typedef PJRT_Error* PJRT_Memory_ToString(PJRT_Memory_ToString_Args* args);

typedef struct PJRT_Memory_AddressableByDevices_Args {
  PJRT_ARGS_HEAD;
  PJRT_Memory* memory;
  PJRT_Device* const* devices; /* out */
  size_t num_devices;          /* out */
} PJRT_Memory_AddressableByDevices_Args;
typedef PJRT_Error* PJRT_Memory_AddressableByDevices(PJRT_Memory_AddressableByDevices_Args* args);

/* ---------------------------------------------------------------- executables (programs.rs:1485-2450) */
typedef struct PJRT_Executable_Destroy_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
} PJRT_Executable_Destroy_Args;
typedef PJRT_Error* PJRT_Executable_Destroy(PJRT_Executable_Destroy_Args* args);

typedef struct PJRT_Executable_Name_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  const char* executable_name; /* out */
  size_t executable_name_size; /* out */
} PJRT_Executable_Name_Args;
typedef PJRT_Error* PJRT_Executable_Name(PJRT_Executable_Name_Args* args);

typedef struct PJRT_Executable_NumReplicas_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  size_t num_replicas; /* out */
} PJRT_Executable_NumReplicas_Args;
typedef PJRT_Error* PJRT_Executable_NumReplicas(PJRT_Executable_NumReplicas_Args* args);

typedef struct PJRT_Executable_NumPartitions_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  size_t num_partitions; /* out */
} PJRT_Executable_NumPartitions_Args;
typedef PJRT_Error* PJRT_Executable_NumPartitions(PJRT_Executable_NumPartitions_Args* args);

typedef struct PJRT_Executable_NumOutputs_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  size_t num_outputs; /* out */
} PJRT_Executable_NumOutputs_Args;
typedef PJRT_Error* PJRT_Executable_NumOutputs(PJRT_Executable_NumOutputs_Args* args);

typedef struct PJRT_Executable_SizeOfGeneratedCodeInBytes_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  int64_t size_in_bytes; /* out */
} PJRT_Executable_SizeOfGeneratedCodeInBytes_Args;
typedef PJRT_Error* PJRT_Executable_SizeOfGeneratedCodeInBytes(PJRT_Executable_SizeOfGeneratedCodeInBytes_Args* args);

typedef struct PJRT_Executable_GetCostAnalysis_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  size_t num_properties;             /* out */
  const PJRT_NamedValue* properties; /* out, owned by the executable */
} PJRT_Executable_GetCostAnalysis_Args;
typedef PJRT_Error* PJRT_Executable_GetCostAnalysis(PJRT_Executable_GetCostAnalysis_Args* args);

typedef struct PJRT_Executable_OutputMemoryKinds_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  size_t num_outputs;               /* out */
  const char* const* memory_kinds;  /* out */
  const size_t* memory_kind_sizes;  /* out */
} PJRT_Executable_OutputMemoryKinds_Args;
typedef PJRT_Error* PJRT_Executable_OutputMemoryKinds(PJRT_Executable_OutputMemoryKinds_Args* args);

typedef struct PJRT_Executable_OptimizedProgram_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  PJRT_Program* program; /* in/out: code==null asks for code_size */
} PJRT_Executable_OptimizedProgram_Args;
typedef PJRT_Error* PJRT_Executable_OptimizedProgram(PJRT_Executable_OptimizedProgram_Args* args);

typedef struct PJRT_Executable_Fingerprint_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  const char* executable_fingerprint; /* out */
  size_t executable_fingerprint_size; /* out */
} PJRT_Executable_Fingerprint_Args;
typedef PJRT_Error* PJRT_Executable_Fingerprint(PJRT_Executable_Fingerprint_Args* args);

typedef struct PJRT_Executable_OutputElementTypes_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  PJRT_Buffer_Type* output_types; /* out */
  size_t num_output_types;        /* out */
} PJRT_Executable_OutputElementTypes_Args;
typedef PJRT_Error* PJRT_Executable_OutputElementTypes(PJRT_Executable_OutputElementTypes_Args* args);

typedef struct PJRT_Executable_OutputDimensions_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  size_t num_outputs;       /* out */
  const int64_t* dims;      /* out: all outputs' dims, concatenated */
  const size_t* dim_sizes;  /* out: rank of each output */
} PJRT_Executable_OutputDimensions_Args;
typedef PJRT_Error* PJRT_Executable_OutputDimensions(PJRT_Executable_OutputDimensions_Args* args);

typedef struct PJRT_Executable_GetCompileOptions_Args {
  PJRT_ARGS_HEAD;
  const PJRT_Executable* executable;
  const char* serialized_bytes;                                     /* out */
  size_t serialized_bytes_size;                                     /* out */
  PJRT_SerializedCompileOptions* serialized_compile_options;        /* out */
  void (*serialized_compile_options_deleter)(PJRT_SerializedCompileOptions* exec); /* out */
} PJRT_Executable_GetCompileOptions_Args;
typedef PJRT_Error* PJRT_Executable_GetCompileOptions(PJRT_Executable_GetCompileOptions_Args* args);

typedef struct PJRT_LoadedExecutable_Destroy_Args {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
} PJRT_LoadedExecutable_Destroy_Args;
typedef PJRT_Error* PJRT_LoadedExecutable_Destroy(PJRT_LoadedExecutable_Destroy_Args* args);

typedef struct PJRT_LoadedExecutable_GetExecutable_Args {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* loaded_executable;
  PJRT_Executable* executable; /* out, caller destroys */
} PJRT_LoadedExecutable_GetExecutable_Args;
typedef PJRT_Error* PJRT_LoadedExecutable_GetExecutable(PJRT_LoadedExecutable_GetExecutable_Args* args);

typedef struct PJRT_LoadedExecutable_AddressableDevices_Args {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
  PJRT_Device* const* addressable_devices; /* out */
  size_t num_addressable_devices;          /* out */
} PJRT_LoadedExecutable_AddressableDevices_Args;
typedef PJRT_Error* PJRT_LoadedExecutable_AddressableDevices(PJRT_LoadedExecutable_AddressableDevices_Args* args);

typedef struct PJRT_LoadedExecutable_Delete_Args {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
} PJRT_LoadedExecutable_Delete_Args;
typedef PJRT_Error* PJRT_LoadedExecutable_Delete(PJRT_LoadedExecutable_Delete_Args* args);

typedef struct PJRT_LoadedExecutable_IsDeleted_Args {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
  bool is_deleted; /* out */
} PJRT_LoadedExecutable_IsDeleted_Args;
typedef PJRT_Error* PJRT_LoadedExecutable_IsDeleted(PJRT_LoadedExecutable_IsDeleted_Args* args);

typedef struct PJRT_LoadedExecutable_Fingerprint_Args {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
  const char* executable_fingerprint; /* out */
  size_t executable_fingerprint_size; /* out */
} PJRT_LoadedExecutable_Fingerprint_Args;
typedef PJRT_Error* PJRT_LoadedExecutable_Fingerprint(PJRT_LoadedExecutable_Fingerprint_Args* args);

typedef struct PJRT_LogicalDeviceIds {
  int replica;
  int partition;
} PJRT_LogicalDeviceIds;

typedef struct PJRT_LoadedExecutable_AddressableDeviceLogicalIds_Args {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
  const PJRT_LogicalDeviceIds* addressable_device_logical_ids; /* out */
  size_t num_addressable_device_logical_ids;                   /* out */
} PJRT_LoadedExecutable_AddressableDeviceLogicalIds_Args;
typedef PJRT_Error* PJRT_LoadedExecutable_AddressableDeviceLogicalIds(
    PJRT_LoadedExecutable_AddressableDeviceLogicalIds_Args* args);

/* Executable_Serialize: programs.rs:1916-1943 (caller: Executable::serialize, programs.rs:404-423). The bytes stay
 * valid until the deleter is called on serialized_executable. */
typedef struct PJRT_Executable_Serialize_Args {
  PJRT_ARGS_HEAD;
  const PJRT_Executable* executable;
  const char* serialized_bytes;                    /* out */
  size_t serialized_bytes_size;                    /* out */
  PJRT_SerializedExecutable* serialized_executable; /* out */
  void (*serialized_executable_deleter)(PJRT_SerializedExecutable* exec); /* out */
} PJRT_Executable_Serialize_Args;
typedef PJRT_Error* PJRT_Executable_Serialize(PJRT_Executable_Serialize_Args* args);

/* Executable_DeserializeAndLoad: programs.rs:2234-2269 (caller: Client::deserialize_and_load_executable,
 * programs.rs:1303-1330). */
typedef struct PJRT_Executable_DeserializeAndLoad_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  const char* serialized_executable;
  size_t serialized_executable_size;
  PJRT_LoadedExecutable* loaded_executable; /* out */
  const char* overridden_serialized_compile_options;
  size_t overridden_serialized_compile_options_size;
} PJRT_Executable_DeserializeAndLoad_Args;
typedef PJRT_Error* PJRT_Executable_DeserializeAndLoad(PJRT_Executable_DeserializeAndLoad_Args* args);

/* LoadedExecutable_GetDeviceAssignment: programs.rs:2052-2080 (caller: LoadedExecutable::device_assignment,
 * programs.rs:704-736). The bytes are a serialized xla.DeviceAssignmentProto (ryft-xla-sys/src/protos.rs:2318-2352). */
typedef struct PJRT_LoadedExecutable_GetDeviceAssignment_Args {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
  const char* serialized_bytes;                                /* out */
  size_t serialized_bytes_size;                                /* out */
  PJRT_DeviceAssignmentSerialized* serialized_device_assignment; /* out */
  void (*serialized_device_assignment_deleter)(PJRT_DeviceAssignmentSerialized* da); /* out */
} PJRT_LoadedExecutable_GetDeviceAssignment_Args;
typedef PJRT_Error* PJRT_LoadedExecutable_GetDeviceAssignment(PJRT_LoadedExecutable_GetDeviceAssignment_Args* args);

/* Executable_GetCompiledMemoryStats: programs.rs (struct PJRT_Executable_GetCompiledMemoryStats_Args; caller
 * Executable::memory_statistics, programs.rs:318-360). */
typedef struct PJRT_Executable_GetCompiledMemoryStats_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  int64_t generated_code_size_in_bytes;      /* out */
  int64_t argument_size_in_bytes;            /* out */
  int64_t output_size_in_bytes;              /* out */
  int64_t alias_size_in_bytes;               /* out */
  int64_t temp_size_in_bytes;                /* out */
  int64_t host_generated_code_size_in_bytes; /* out */
  int64_t host_argument_size_in_bytes;       /* out */
  int64_t host_output_size_in_bytes;         /* out */
  int64_t host_alias_size_in_bytes;          /* out */
  int64_t host_temp_size_in_bytes;           /* out */
  int64_t peak_memory_in_bytes;              /* out */
  int64_t total_size_in_bytes;               /* out */
  int64_t total_allocation_bytes;            /* out */
  int64_t indefinite_allocations;            /* out */
  int64_t peak_unpadded_heap_bytes;          /* out */
} PJRT_Executable_GetCompiledMemoryStats_Args;
typedef PJRT_Error* PJRT_Executable_GetCompiledMemoryStats(PJRT_Executable_GetCompiledMemoryStats_Args* args);

/* Executable_ParameterMemoryKinds: programs.rs:1606-1630 (caller: Executable::input_memory_kinds, programs.rs:127-145). */
typedef struct PJRT_Executable_ParameterMemoryKinds_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  size_t num_parameters;             /* out */
  const char* const* memory_kinds;   /* out */
  const size_t* memory_kind_sizes;   /* out */
} PJRT_Executable_ParameterMemoryKinds_Args;
typedef PJRT_Error* PJRT_Executable_ParameterMemoryKinds(PJRT_Executable_ParameterMemoryKinds_Args* args);

/* ExecuteContext_Create / _Destroy: programs.rs:2311-2345 (caller: Api::execution_context, programs.rs:1476-1481). */
typedef struct PJRT_ExecuteContext_Create_Args {
  PJRT_ARGS_HEAD;
  PJRT_ExecuteContext* context; /* out */
} PJRT_ExecuteContext_Create_Args;
typedef PJRT_Error* PJRT_ExecuteContext_Create(PJRT_ExecuteContext_Create_Args* args);
typedef struct PJRT_ExecuteContext_Destroy_Args {
  PJRT_ARGS_HEAD;
  PJRT_ExecuteContext* context;
} PJRT_ExecuteContext_Destroy_Args;
typedef PJRT_Error* PJRT_ExecuteContext_Destroy(PJRT_ExecuteContext_Destroy_Args* args);

typedef struct PJRT_SendCallbackInfo PJRT_SendCallbackInfo;
typedef struct PJRT_RecvCallbackInfo PJRT_RecvCallbackInfo;

typedef struct PJRT_ExecuteOptions {
  PJRT_ARGS_HEAD;
  PJRT_SendCallbackInfo** send_callbacks;
  PJRT_RecvCallbackInfo** recv_callbacks;
  size_t num_send_ops;
  size_t num_recv_ops;
  int launch_id;
  const int64_t* non_donatable_input_indices;
  size_t num_non_donatable_input_indices;
  PJRT_ExecuteContext* context;
  const char* call_location;
  size_t num_tasks;
  int* task_ids;
  int64_t* incarnation_ids;
  PJRT_MultiSlice_Config* multi_slice_config;
} PJRT_ExecuteOptions;

typedef struct PJRT_LoadedExecutable_Execute_Args {
  PJRT_ARGS_HEAD;
  PJRT_LoadedExecutable* executable;
  PJRT_ExecuteOptions* options;
  PJRT_Buffer* const* const* argument_lists; /* [num_devices][num_args] */
  size_t num_devices;
  size_t num_args;
  PJRT_Buffer** const* output_lists;  /* [num_devices][num_outputs], filled */
  PJRT_Event** device_complete_events; /* [num_devices], filled (may be null) */
  PJRT_Device* execute_device;
} PJRT_LoadedExecutable_Execute_Args;
typedef PJRT_Error* PJRT_LoadedExecutable_Execute(PJRT_LoadedExecutable_Execute_Args* args);

/* ---------------------------------------------------------------- layouts extension (extensions/layouts.rs:590-808) */
/* Version 4 (PJRT_API_LAYOUTS_EXTENSION_VERSION, layouts.rs:599), type PJRT_Extension_Type_Layouts. Layouts returned
 * by Client_GetDefaultLayout and Buffer_MemoryLayout belong to the caller (MemoryLayout_Destroy); those returned by
 * the executable functions belong to the executable (layouts.rs:245-290 marks them borrowed). */
typedef struct PJRT_Layouts_MemoryLayout PJRT_Layouts_MemoryLayout;
typedef struct PJRT_Layouts_SerializedLayout PJRT_Layouts_SerializedLayout;

typedef struct PJRT_Layouts_MemoryLayout_Destroy_Args {
  PJRT_ARGS_HEAD;
  PJRT_Layouts_MemoryLayout* layout;
} PJRT_Layouts_MemoryLayout_Destroy_Args;
typedef PJRT_Error* PJRT_Layouts_MemoryLayout_Destroy(PJRT_Layouts_MemoryLayout_Destroy_Args* args);

typedef struct PJRT_Layouts_MemoryLayout_Serialize_Args {
  PJRT_ARGS_HEAD;
  PJRT_Layouts_MemoryLayout* layout;
  const char* serialized_bytes;                      /* out */
  size_t serialized_bytes_size;                      /* out */
  PJRT_Layouts_SerializedLayout* serialized_layout;  /* out */
  void (*serialized_layout_deleter)(PJRT_Layouts_SerializedLayout* s_layout); /* out */
} PJRT_Layouts_MemoryLayout_Serialize_Args;
typedef PJRT_Error* PJRT_Layouts_MemoryLayout_Serialize(PJRT_Layouts_MemoryLayout_Serialize_Args* args);

typedef struct PJRT_Layouts_PJRT_Client_GetDefaultLayout_Args {
  PJRT_ARGS_HEAD;
  PJRT_Client* client;
  PJRT_Buffer_Type element_type;
  const int64_t* dims;
  size_t num_dims;
  PJRT_Layouts_MemoryLayout* layout; /* out */
} PJRT_Layouts_PJRT_Client_GetDefaultLayout_Args;
typedef PJRT_Error* PJRT_Layouts_PJRT_Client_GetDefaultLayout(PJRT_Layouts_PJRT_Client_GetDefaultLayout_Args* args);

typedef struct PJRT_Layouts_PJRT_Buffer_MemoryLayout_Args {
  PJRT_ARGS_HEAD;
  PJRT_Buffer* buffer;
  PJRT_Layouts_MemoryLayout* layout; /* out */
} PJRT_Layouts_PJRT_Buffer_MemoryLayout_Args;
typedef PJRT_Error* PJRT_Layouts_PJRT_Buffer_MemoryLayout(PJRT_Layouts_PJRT_Buffer_MemoryLayout_Args* args);

typedef struct PJRT_Layouts_PJRT_Executable_GetOutputLayouts_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  size_t num_outputs;                    /* out */
  PJRT_Layouts_MemoryLayout** layouts;   /* out */
} PJRT_Layouts_PJRT_Executable_GetOutputLayouts_Args;
typedef PJRT_Error* PJRT_Layouts_PJRT_Executable_GetOutputLayouts(PJRT_Layouts_PJRT_Executable_GetOutputLayouts_Args* args);

typedef struct PJRT_Layouts_PJRT_Executable_GetParameterLayouts_Args {
  PJRT_ARGS_HEAD;
  PJRT_Executable* executable;
  size_t num_parameters;                 /* out */
  PJRT_Layouts_MemoryLayout** layouts;   /* out */
} PJRT_Layouts_PJRT_Executable_GetParameterLayouts_Args;
typedef PJRT_Error* PJRT_Layouts_PJRT_Executable_GetParameterLayouts(
    PJRT_Layouts_PJRT_Executable_GetParameterLayouts_Args* args);

#define PJRT_API_LAYOUTS_EXTENSION_VERSION 4
typedef struct PJRT_Layouts_Extension {
  PJRT_Extension_Base base;
  PJRT_Layouts_MemoryLayout_Destroy* PJRT_Layouts_MemoryLayout_Destroy;
  PJRT_Layouts_MemoryLayout_Serialize* PJRT_Layouts_MemoryLayout_Serialize;
  PJRT_Layouts_PJRT_Client_GetDefaultLayout* PJRT_Layouts_PJRT_Client_GetDefaultLayout;
  PJRT_Layouts_PJRT_Buffer_MemoryLayout* PJRT_Layouts_PJRT_Buffer_MemoryLayout;
  PJRT_Unimplemented_Fn PJRT_Layouts_PJRT_Topology_GetDefaultLayout; /* no topology descriptions */
  PJRT_Layouts_PJRT_Executable_GetOutputLayouts* PJRT_Layouts_PJRT_Executable_GetOutputLayouts;
  PJRT_Layouts_PJRT_Executable_GetParameterLayouts* PJRT_Layouts_PJRT_Executable_GetParameterLayouts;
} PJRT_Layouts_Extension;

/* ---------------------------------------------------------------- memory descriptions extension
 * (extensions/memory_descriptions.rs:209-285; version 1, type PJRT_Extension_Type_MemoryDescriptions) */
typedef struct PJRT_MemoryDescription PJRT_MemoryDescription;

typedef struct PJRT_DeviceDescription_MemoryDescriptions_Args {
  PJRT_ARGS_HEAD;
  PJRT_DeviceDescription* device_description;
  const PJRT_MemoryDescription* const* memory_descriptions; /* out, owned by the description */
  size_t num_memory_descriptions;                           /* out */
  ptrdiff_t default_memory_index;                           /* out; -1: none */
} PJRT_DeviceDescription_MemoryDescriptions_Args;
typedef PJRT_Error* PJRT_DeviceDescription_MemoryDescriptions(PJRT_DeviceDescription_MemoryDescriptions_Args* args);

typedef struct PJRT_MemoryDescription_Kind_Args {
  PJRT_ARGS_HEAD;
  const PJRT_MemoryDescription* memory_description;
  const char* kind;  /* out */
  size_t kind_size;  /* out */
  int kind_id;       /* out */
} PJRT_MemoryDescription_Kind_Args;
typedef PJRT_Error* PJRT_MemoryDescription_Kind(PJRT_MemoryDescription_Kind_Args* args);

#define PJRT_API_MEMORY_DESCRIPTIONS_EXTENSION_VERSION 1
typedef struct PJRT_MemoryDescriptions_Extension {
  PJRT_Extension_Base base;
  PJRT_DeviceDescription_MemoryDescriptions* PJRT_DeviceDescription_MemoryDescriptions;
  PJRT_MemoryDescription_Kind* PJRT_MemoryDescription_Kind;
} PJRT_MemoryDescriptions_Extension;

/* ---------------------------------------------------------------- profiler extension (extensions/profiler.rs:345-520)
 * Errors of this API are its own type (PLUGIN_Profiler_Error), released with its own Error_Destroy. */
#define PJRT_API_PROFILER_EXTENSION_VERSION 1
typedef struct PLUGIN_Profiler_Error PLUGIN_Profiler_Error;
typedef struct PLUGIN_Profiler PLUGIN_Profiler;

typedef struct PLUGIN_Profiler_Error_Message_Args {
  size_t struct_size;
  void* state;
  const PLUGIN_Profiler_Error* error;
  const char* message; /* out */
  size_t message_size; /* out */
} PLUGIN_Profiler_Error_Message_Args;
typedef void PLUGIN_Profiler_Error_Message(PLUGIN_Profiler_Error_Message_Args* args);

typedef struct PLUGIN_Profiler_Error_GetCode_Args {
  size_t struct_size;
  void* state;
  const PLUGIN_Profiler_Error* error;
  int code; /* out */
} PLUGIN_Profiler_Error_GetCode_Args;
typedef PLUGIN_Profiler_Error* PLUGIN_Profiler_Error_GetCode(PLUGIN_Profiler_Error_GetCode_Args* args);

typedef struct PLUGIN_Profiler_Error_Destroy_Args {
  size_t struct_size;
  void* state;
  PLUGIN_Profiler_Error* error;
} PLUGIN_Profiler_Error_Destroy_Args;
typedef void PLUGIN_Profiler_Error_Destroy(PLUGIN_Profiler_Error_Destroy_Args* args);

typedef struct PLUGIN_Profiler_Create_Args {
  size_t struct_size;
  const char* options; /* serialized tensorflow.ProfileOptions */
  size_t options_size;
  PLUGIN_Profiler* profiler; /* out */
} PLUGIN_Profiler_Create_Args;
typedef PLUGIN_Profiler_Error* PLUGIN_Profiler_Create(PLUGIN_Profiler_Create_Args* args);

typedef struct PLUGIN_Profiler_Destroy_Args {
  size_t struct_size;
  PLUGIN_Profiler* profiler;
} PLUGIN_Profiler_Destroy_Args;
typedef PLUGIN_Profiler_Error* PLUGIN_Profiler_Destroy(PLUGIN_Profiler_Destroy_Args* args);

typedef struct PLUGIN_Profiler_Start_Args {
  size_t struct_size;
  PLUGIN_Profiler* profiler;
} PLUGIN_Profiler_Start_Args;
typedef PLUGIN_Profiler_Error* PLUGIN_Profiler_Start(PLUGIN_Profiler_Start_Args* args);

typedef struct PLUGIN_Profiler_Stop_Args {
  size_t struct_size;
  PLUGIN_Profiler* profiler;
} PLUGIN_Profiler_Stop_Args;
typedef PLUGIN_Profiler_Error* PLUGIN_Profiler_Stop(PLUGIN_Profiler_Stop_Args* args);

/* A call with a null buffer serializes the session's XSpace into storage the session owns (valid until Destroy) and
 * returns it with its size (one trailing NUL included); a call with a non-null buffer does nothing. */
typedef struct PLUGIN_Profiler_CollectData_Args {
  size_t struct_size;
  PLUGIN_Profiler* profiler;
  uint8_t* buffer;             /* in/out */
  size_t buffer_size_in_bytes; /* out */
} PLUGIN_Profiler_CollectData_Args;
typedef PLUGIN_Profiler_Error* PLUGIN_Profiler_CollectData(PLUGIN_Profiler_CollectData_Args* args);

typedef struct PLUGIN_Profiler_Api {
  size_t struct_size;
  void* state;
  PLUGIN_Profiler_Error_Destroy* PLUGIN_Profiler_Error_Destroy;
  PLUGIN_Profiler_Error_Message* PLUGIN_Profiler_Error_Message;
  PLUGIN_Profiler_Error_GetCode* PLUGIN_Profiler_Error_GetCode;
  PLUGIN_Profiler_Create* PLUGIN_Profiler_Create;
  PLUGIN_Profiler_Destroy* PLUGIN_Profiler_Destroy;
  PLUGIN_Profiler_Start* PLUGIN_Profiler_Start;
  PLUGIN_Profiler_Stop* PLUGIN_Profiler_Stop;
  PLUGIN_Profiler_CollectData* PLUGIN_Profiler_CollectData;
} PLUGIN_Profiler_Api;

typedef struct PJRT_Profiler_Extension {
  PJRT_Extension_Base base;
  PLUGIN_Profiler_Api* profiler_api;
  int64_t trace_me_context_id;
} PJRT_Profiler_Extension;

/* ---------------------------------------------------------------- the table (lib.rs:214-364) */
#define PJRT_SLOT(name) name* name
#define PJRT_NOSLOT(name) PJRT_Unimplemented_Fn name

typedef struct PJRT_Api {
  size_t struct_size;
  PJRT_Extension_Base* extension_start;
  PJRT_Api_Version pjrt_api_version;

  PJRT_SLOT(PJRT_Error_Destroy);
  PJRT_SLOT(PJRT_Error_Message);
  PJRT_SLOT(PJRT_Error_GetCode);
  PJRT_SLOT(PJRT_Plugin_Initialize);
  PJRT_SLOT(PJRT_Plugin_Attributes);
  PJRT_SLOT(PJRT_Event_Destroy);
  PJRT_SLOT(PJRT_Event_IsReady);
  PJRT_SLOT(PJRT_Event_Error);
  PJRT_SLOT(PJRT_Event_Await);
  PJRT_SLOT(PJRT_Event_OnReady);
  PJRT_SLOT(PJRT_Client_Create);
  PJRT_SLOT(PJRT_Client_Destroy);
  PJRT_SLOT(PJRT_Client_PlatformName);
  PJRT_SLOT(PJRT_Client_ProcessIndex);
  PJRT_SLOT(PJRT_Client_PlatformVersion);
  PJRT_SLOT(PJRT_Client_Devices);
  PJRT_SLOT(PJRT_Client_AddressableDevices);
  PJRT_SLOT(PJRT_Client_LookupDevice);
  PJRT_SLOT(PJRT_Client_LookupAddressableDevice);
  PJRT_SLOT(PJRT_Client_AddressableMemories);
  PJRT_SLOT(PJRT_Client_Compile);
  PJRT_SLOT(PJRT_Client_DefaultDeviceAssignment);
  PJRT_SLOT(PJRT_Client_BufferFromHostBuffer);
  PJRT_SLOT(PJRT_DeviceDescription_Id);
  PJRT_SLOT(PJRT_DeviceDescription_ProcessIndex);
  PJRT_SLOT(PJRT_DeviceDescription_Attributes);
  PJRT_SLOT(PJRT_DeviceDescription_Kind);
  PJRT_SLOT(PJRT_DeviceDescription_DebugString);
  PJRT_SLOT(PJRT_DeviceDescription_ToString);
  PJRT_SLOT(PJRT_Device_GetDescription);
  PJRT_SLOT(PJRT_Device_IsAddressable);
  PJRT_SLOT(PJRT_Device_LocalHardwareId);
  PJRT_SLOT(PJRT_Device_AddressableMemories);
  PJRT_SLOT(PJRT_Device_DefaultMemory);
  PJRT_SLOT(PJRT_Device_MemoryStats);
  PJRT_SLOT(PJRT_Memory_Id);
  PJRT_SLOT(PJRT_Memory_Kind);
  PJRT_SLOT(PJRT_Memory_DebugString);
  PJRT_SLOT(PJRT_Memory_ToString);
  PJRT_SLOT(PJRT_Memory_AddressableByDevices);
  PJRT_SLOT(PJRT_Executable_Destroy);
  PJRT_SLOT(PJRT_Executable_Name);
  PJRT_SLOT(PJRT_Executable_NumReplicas);
  PJRT_SLOT(PJRT_Executable_NumPartitions);
  PJRT_SLOT(PJRT_Executable_NumOutputs);
  PJRT_SLOT(PJRT_Executable_SizeOfGeneratedCodeInBytes);
  PJRT_SLOT(PJRT_Executable_GetCostAnalysis);
  PJRT_SLOT(PJRT_Executable_OutputMemoryKinds);
  PJRT_SLOT(PJRT_Executable_OptimizedProgram);
  PJRT_SLOT(PJRT_Executable_Serialize);
  PJRT_SLOT(PJRT_LoadedExecutable_Destroy);
  PJRT_SLOT(PJRT_LoadedExecutable_GetExecutable);
  PJRT_SLOT(PJRT_LoadedExecutable_AddressableDevices);
  PJRT_SLOT(PJRT_LoadedExecutable_Delete);
  PJRT_SLOT(PJRT_LoadedExecutable_IsDeleted);
  PJRT_SLOT(PJRT_LoadedExecutable_Execute);
  PJRT_SLOT(PJRT_Executable_DeserializeAndLoad);
  PJRT_SLOT(PJRT_LoadedExecutable_Fingerprint);
  PJRT_SLOT(PJRT_Buffer_Destroy);
  PJRT_SLOT(PJRT_Buffer_ElementType);
  PJRT_SLOT(PJRT_Buffer_Dimensions);
  PJRT_SLOT(PJRT_Buffer_UnpaddedDimensions);
  PJRT_SLOT(PJRT_Buffer_DynamicDimensionIndices);
  PJRT_SLOT(PJRT_Buffer_GetMemoryLayout);
  PJRT_SLOT(PJRT_Buffer_OnDeviceSizeInBytes);
  PJRT_SLOT(PJRT_Buffer_Device);
  PJRT_SLOT(PJRT_Buffer_Memory);
  PJRT_SLOT(PJRT_Buffer_Delete);
  PJRT_SLOT(PJRT_Buffer_IsDeleted);
  PJRT_SLOT(PJRT_Buffer_CopyToDevice);
  PJRT_SLOT(PJRT_Buffer_ToHostBuffer);
  PJRT_SLOT(PJRT_Buffer_IsOnCpu);
  PJRT_SLOT(PJRT_Buffer_ReadyEvent);
  PJRT_SLOT(PJRT_Buffer_UnsafePointer);
  PJRT_SLOT(PJRT_Buffer_IncreaseExternalReferenceCount);
  PJRT_SLOT(PJRT_Buffer_DecreaseExternalReferenceCount);
  PJRT_SLOT(PJRT_Buffer_OpaqueDeviceMemoryDataPointer);
  PJRT_NOSLOT(PJRT_CopyToDeviceStream_Destroy);
  PJRT_NOSLOT(PJRT_CopyToDeviceStream_AddChunk);
  PJRT_NOSLOT(PJRT_CopyToDeviceStream_TotalBytes);
  PJRT_NOSLOT(PJRT_CopyToDeviceStream_GranuleSize);
  PJRT_NOSLOT(PJRT_CopyToDeviceStream_CurrentBytes);
  PJRT_NOSLOT(PJRT_TopologyDescription_Create);
  PJRT_NOSLOT(PJRT_TopologyDescription_Destroy);
  PJRT_NOSLOT(PJRT_TopologyDescription_PlatformName);
  PJRT_NOSLOT(PJRT_TopologyDescription_PlatformVersion);
  PJRT_NOSLOT(PJRT_TopologyDescription_GetDeviceDescriptions);
  PJRT_NOSLOT(PJRT_TopologyDescription_Serialize);
  PJRT_NOSLOT(PJRT_TopologyDescription_Attributes);
  PJRT_NOSLOT(PJRT_Compile);
  PJRT_SLOT(PJRT_Executable_OutputElementTypes);
  PJRT_SLOT(PJRT_Executable_OutputDimensions);
  PJRT_SLOT(PJRT_Buffer_CopyToMemory);
  PJRT_NOSLOT(PJRT_Client_CreateViewOfDeviceBuffer);
  PJRT_SLOT(PJRT_Executable_Fingerprint);
  PJRT_NOSLOT(PJRT_Client_TopologyDescription);
  PJRT_SLOT(PJRT_Executable_GetCompiledMemoryStats);
  PJRT_SLOT(PJRT_Memory_Kind_Id);
  PJRT_SLOT(PJRT_ExecuteContext_Create);
  PJRT_SLOT(PJRT_ExecuteContext_Destroy);
  PJRT_SLOT(PJRT_Buffer_CopyRawToHost);
  PJRT_NOSLOT(PJRT_AsyncHostToDeviceTransferManager_Destroy);
  PJRT_NOSLOT(PJRT_AsyncHostToDeviceTransferManager_TransferData);
  PJRT_NOSLOT(PJRT_Client_CreateBuffersForAsyncHostToDevice);
  PJRT_NOSLOT(PJRT_AsyncHostToDeviceTransferManager_RetrieveBuffer);
  PJRT_NOSLOT(PJRT_AsyncHostToDeviceTransferManager_Device);
  PJRT_NOSLOT(PJRT_AsyncHostToDeviceTransferManager_BufferCount);
  PJRT_NOSLOT(PJRT_AsyncHostToDeviceTransferManager_BufferSize);
  PJRT_NOSLOT(PJRT_AsyncHostToDeviceTransferManager_SetBufferError);
  PJRT_NOSLOT(PJRT_AsyncHostToDeviceTransferManager_AddMetadata);
  PJRT_NOSLOT(PJRT_Client_DmaMap);
  PJRT_NOSLOT(PJRT_Client_DmaUnmap);
  PJRT_SLOT(PJRT_Client_CreateUninitializedBuffer);
  PJRT_NOSLOT(PJRT_Client_UpdateGlobalProcessInfo);
  PJRT_NOSLOT(PJRT_TopologyDescription_Deserialize);
  PJRT_NOSLOT(PJRT_Client_CreateAliasBuffer);
  PJRT_NOSLOT(PJRT_Client_FulfillAliasBuffer);
  PJRT_SLOT(PJRT_LoadedExecutable_GetDeviceAssignment);
  PJRT_SLOT(PJRT_Client_CreateErrorBuffer);
  PJRT_NOSLOT(PJRT_AsyncHostToDeviceTransferManager_TransferLiteral);
  PJRT_NOSLOT(PJRT_Buffer_CopyRawToHostFuture);
  PJRT_SLOT(PJRT_Device_PoisonExecution);
  PJRT_NOSLOT(PJRT_Device_CreateAsyncTrackingEvent);
  PJRT_NOSLOT(PJRT_AsyncTrackingEvent_Destroy);
  PJRT_SLOT(PJRT_Executable_GetCompileOptions);
  PJRT_NOSLOT(PJRT_Buffer_DonateWithControlDependency);
  PJRT_SLOT(PJRT_Event_Create);
  PJRT_SLOT(PJRT_Event_Set);
  PJRT_NOSLOT(PJRT_Device_GetAttributes);
  PJRT_NOSLOT(PJRT_Client_Load);
  PJRT_SLOT(PJRT_LoadedExecutable_AddressableDeviceLogicalIds);
  PJRT_NOSLOT(PJRT_Buffer_Bitcast);
  PJRT_SLOT(PJRT_Error_ForEachPayload);
  PJRT_NOSLOT(PJRT_TopologyDescription_Fingerprint);
  PJRT_SLOT(PJRT_Executable_ParameterMemoryKinds);
} PJRT_Api;

#undef PJRT_SLOT
#undef PJRT_NOSLOT

/* ---------------------------------------------------------------- layout checks (hand-computed, LP64) */
#if defined(__cplusplus)
#define PJRT_ASSERT(c, m) static_assert(c, m)
#else
#define PJRT_ASSERT(c, m) _Static_assert(c, m)
#endif
PJRT_ASSERT(sizeof(PJRT_Extension_Base) == 24, "PJRT_Extension_Base");
PJRT_ASSERT(sizeof(PJRT_Api_Version) == 24, "PJRT_Api_Version");
PJRT_ASSERT(offsetof(PJRT_Api, PJRT_Error_Destroy) == 40, "first PJRT_Api slot");
/* 3 header fields (8+8+24 bytes) + 135 function slots of 8 bytes. */
PJRT_ASSERT(sizeof(PJRT_Api) == 40 + 135 * 8, "PJRT_Api has 135 slots");
PJRT_ASSERT(offsetof(PJRT_Api, PJRT_LoadedExecutable_Execute) == 40 + 55 * 8, "Execute slot");
PJRT_ASSERT(offsetof(PJRT_Api, PJRT_Executable_ParameterMemoryKinds) == 40 + 134 * 8, "last slot");
PJRT_ASSERT(sizeof(PJRT_NamedValue) == 56, "PJRT_NamedValue");
PJRT_ASSERT(offsetof(PJRT_NamedValue, value_size) == 48, "PJRT_NamedValue.value_size");
PJRT_ASSERT(sizeof(PJRT_Client_Create_Args) == 88, "PJRT_Client_Create_Args");
PJRT_ASSERT(offsetof(PJRT_Client_Create_Args, client) == 64, "PJRT_Client_Create_Args.client");
PJRT_ASSERT(sizeof(PJRT_Program) == 48, "PJRT_Program");
PJRT_ASSERT(sizeof(PJRT_Client_Compile_Args) == 56, "PJRT_Client_Compile_Args");
PJRT_ASSERT(sizeof(PJRT_Buffer_MemoryLayout_Tiled) == 56, "Tiled layout");
PJRT_ASSERT(sizeof(PJRT_Buffer_MemoryLayout) == 80, "PJRT_Buffer_MemoryLayout");
PJRT_ASSERT(offsetof(PJRT_Buffer_MemoryLayout, type) == 72, "PJRT_Buffer_MemoryLayout.type");
PJRT_ASSERT(sizeof(PJRT_Buffer_GetMemoryLayout_Args) == 104, "PJRT_Buffer_GetMemoryLayout_Args");
PJRT_ASSERT(sizeof(PJRT_Client_BufferFromHostBuffer_Args) == 120, "PJRT_Client_BufferFromHostBuffer_Args");
PJRT_ASSERT(offsetof(PJRT_Client_BufferFromHostBuffer_Args, type) == 32, "BufferFromHostBuffer.type");
PJRT_ASSERT(sizeof(PJRT_Client_CreateErrorBuffer_Args) == 112, "PJRT_Client_CreateErrorBuffer_Args");
PJRT_ASSERT(offsetof(PJRT_Client_CreateErrorBuffer_Args, shape_element_type) == 64, "CreateErrorBuffer.type");
PJRT_ASSERT(offsetof(PJRT_Client_CreateErrorBuffer_Args, buffer) == 88, "CreateErrorBuffer.buffer");
PJRT_ASSERT(sizeof(PJRT_Device_PoisonExecution_Args) == 72, "PJRT_Device_PoisonExecution_Args");
PJRT_ASSERT(offsetof(PJRT_Device_PoisonExecution_Args, error_code) == 28, "PoisonExecution.error_code");
PJRT_ASSERT(offsetof(PJRT_Device_PoisonExecution_Args, poisoned) == 48, "PoisonExecution.poisoned");
PJRT_ASSERT(offsetof(PJRT_Client_BufferFromHostBuffer_Args, host_buffer_semantics) == 72, "semantics");
PJRT_ASSERT(offsetof(PJRT_Client_BufferFromHostBuffer_Args, buffer) == 112, "BufferFromHostBuffer.buffer");
PJRT_ASSERT(sizeof(PJRT_Buffer_ToHostBuffer_Args) == 56, "PJRT_Buffer_ToHostBuffer_Args");
PJRT_ASSERT(sizeof(PJRT_ExecuteOptions) == 120, "PJRT_ExecuteOptions");
PJRT_ASSERT(offsetof(PJRT_ExecuteOptions, launch_id) == 48, "PJRT_ExecuteOptions.launch_id");
PJRT_ASSERT(sizeof(PJRT_LoadedExecutable_Execute_Args) == 80, "PJRT_LoadedExecutable_Execute_Args");
PJRT_ASSERT(sizeof(PJRT_Event_Set_Args) == 48, "PJRT_Event_Set_Args");
PJRT_ASSERT(sizeof(PJRT_Device_MemoryStats_Args) == 192, "PJRT_Device_MemoryStats_Args");
PJRT_ASSERT(sizeof(PJRT_Executable_OutputDimensions_Args) == 48, "PJRT_Executable_OutputDimensions_Args");
PJRT_ASSERT(sizeof(PJRT_Executable_GetCompileOptions_Args) == 56, "PJRT_Executable_GetCompileOptions_Args");
PJRT_ASSERT(sizeof(PJRT_Executable_Serialize_Args) == 56, "PJRT_Executable_Serialize_Args");
PJRT_ASSERT(sizeof(PJRT_Layouts_Extension) == 24 + 7 * 8, "PJRT_Layouts_Extension");
PJRT_ASSERT(sizeof(PJRT_MemoryDescriptions_Extension) == 24 + 2 * 8, "PJRT_MemoryDescriptions_Extension");
PJRT_ASSERT(sizeof(PJRT_Profiler_Extension) == 24 + 2 * 8, "PJRT_Profiler_Extension");
PJRT_ASSERT(sizeof(PLUGIN_Profiler_Api) == 10 * 8, "PLUGIN_Profiler_Api");
PJRT_ASSERT(sizeof(PLUGIN_Profiler_Error_Message_Args) == 40, "PLUGIN_Profiler_Error_Message_Args");
PJRT_ASSERT(sizeof(PLUGIN_Profiler_Error_GetCode_Args) == 32, "PLUGIN_Profiler_Error_GetCode_Args");
PJRT_ASSERT(sizeof(PLUGIN_Profiler_Create_Args) == 32, "PLUGIN_Profiler_Create_Args");
PJRT_ASSERT(sizeof(PLUGIN_Profiler_CollectData_Args) == 32, "PLUGIN_Profiler_CollectData_Args");
PJRT_ASSERT(sizeof(PJRT_DeviceDescription_MemoryDescriptions_Args) == 48, "MemoryDescriptions_Args");
PJRT_ASSERT(sizeof(PJRT_MemoryDescription_Kind_Args) == 48, "PJRT_MemoryDescription_Kind_Args");
PJRT_ASSERT(sizeof(PJRT_Layouts_PJRT_Client_GetDefaultLayout_Args) == 56, "PJRT_Layouts_PJRT_Client_GetDefaultLayout_Args");
PJRT_ASSERT(offsetof(PJRT_Layouts_PJRT_Client_GetDefaultLayout_Args, dims) == 32, "GetDefaultLayout.dims");
PJRT_ASSERT(sizeof(PJRT_Layouts_MemoryLayout_Serialize_Args) == 56, "PJRT_Layouts_MemoryLayout_Serialize_Args");
PJRT_ASSERT(sizeof(PJRT_Layouts_PJRT_Executable_GetOutputLayouts_Args) == 40, "GetOutputLayouts_Args");
PJRT_ASSERT(sizeof(PJRT_Executable_DeserializeAndLoad_Args) == 64, "PJRT_Executable_DeserializeAndLoad_Args");
PJRT_ASSERT(offsetof(PJRT_Executable_DeserializeAndLoad_Args, loaded_executable) == 40,
            "PJRT_Executable_DeserializeAndLoad_Args.loaded_executable");
PJRT_ASSERT(sizeof(PJRT_LoadedExecutable_GetDeviceAssignment_Args) == 56, "PJRT_LoadedExecutable_GetDeviceAssignment_Args");
PJRT_ASSERT(sizeof(PJRT_Executable_GetCompiledMemoryStats_Args) == 144, "PJRT_Executable_GetCompiledMemoryStats_Args");
PJRT_ASSERT(offsetof(PJRT_Executable_GetCompiledMemoryStats_Args, peak_memory_in_bytes) == 104,
            "PJRT_Executable_GetCompiledMemoryStats_Args.peak_memory_in_bytes");
PJRT_ASSERT(sizeof(PJRT_Executable_ParameterMemoryKinds_Args) == 48, "PJRT_Executable_ParameterMemoryKinds_Args");
PJRT_ASSERT(sizeof(PJRT_ExecuteContext_Create_Args) == 24, "PJRT_ExecuteContext_Create_Args");
PJRT_ASSERT(sizeof(PJRT_Buffer_CopyRawToHost_Args) == 56, "PJRT_Buffer_CopyRawToHost_Args");
#undef PJRT_ASSERT

#ifdef __cplusplus
}
#endif

#endif /* RYFT_MI355X_PJRT_C_API_H_ */
