/*
 * ryft MI355X PJRT plugin — the C-ABI entry point and the plugin's own extension.
 *
 * The plugin exports exactly one symbol, GetPjrtApi, which ryft-pjrt resolves with libloading from
 * `load_plugin(path)` (crates/ryft-pjrt/src/plugins.rs:67-80, 120-122) and whose signature is the one ryft-xla-sys
 * binds for the statically linked XLA CPU plugin (crates/ryft-xla-sys/src/bindings.rs:10). The export list mirrors
 * crates/ryft-xla-sys/pjrt_plugin_version_script.lds. The returned table is static, immutable, and identical on
 * every call.
 */
#ifndef RYFT_MI355X_H_
#define RYFT_MI355X_H_

#include "pjrt_c_api.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces ryft_xla_sys::bindings::GetPjrtApi (crates/ryft-xla-sys/src/bindings.rs:10) behind load_plugin(). */
const PJRT_Api* GetPjrtApi(void);

/*
 * Plugin extension, reachable by walking PJRT_Api.extension_start (the same walk ryft-pjrt performs for its known
 * extensions, crates/ryft-pjrt/src/extensions/layouts.rs:78-92). Its type tag is outside the PJRT_Extension_Type
 * range, so callers that do not know it skip it. It has no counterpart in the reference: it exposes per-kernel
 * timing measured with HIP events on the device stream, and the fused plan of a loaded executable.
 */
#define RYFT_MI355X_EXTENSION_TYPE 0x52594654u /* 'RYFT' */

typedef struct RYFT_MI355X_Extension {
  PJRT_Extension_Base base;
  /* Turn per-kernel HIP-event timing on or off for every execution on `client`. */
  PJRT_Error* (*set_kernel_timing)(PJRT_Client* client, bool enable);
  /* Synchronize the device and return a JSON object {kernel: {count, total_ms, avg_us, min_us, max_us, flops,
   * bytes}} aggregated since the last call (then reset). The string stays valid until the next call. */
  PJRT_Error* (*kernel_timing)(PJRT_Client* client, const char** json, size_t* json_size);
  /* Human-readable fused plan (one line per kernel launch). Valid while the executable lives. */
  PJRT_Error* (*describe_plan)(PJRT_LoadedExecutable* executable, const char** text, size_t* text_size);
} RYFT_MI355X_Extension;

/*
 * Allocation-free execution. No counterpart in the reference (ryft-pjrt's execute path is
 * PJRT_LoadedExecutable_Execute, crates/ryft-pjrt/src/programs.rs:769-963, which allocates its results); it is for
 * callers that cannot allocate device memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.
 *
 * Enqueues one execution of `executable` (a PJRT_LoadedExecutable of this plugin, on its first device) on `stream`
 * (a hipStream_t of that device; null = the device's null stream) and returns without waiting. The caller passes
 * the device memory of every parameter (`inputs[i]`, `input_sizes[i]` bytes, dense row-major) and every result
 * (`outputs[o]`, `output_sizes[o]` bytes); sizes must equal the program's and pointers be 256-byte aligned. The
 * plan's intermediates live in a per-GPU scratch array of 64 MiB that the library holds until the process ends;
 * an executable needing more is rejected with RESOURCE_EXHAUSTED. Nothing is allocated on the device (no hipMalloc,
 * no hipFree) and no event is created. Calls that overlap on one GPU share that scratch and race; the caller orders
 * the producers of the inputs before the call and waits on `stream` before reading the outputs.
 *
 * Returns 0 on success, else a PJRT_Error_Code; `*error_message` (if non-null) then points at a description that
 * stays valid until the calling thread's next call.
 */
int RyftMi355x_ExecuteNoAlloc(PJRT_LoadedExecutable* executable, const void* const* inputs, const size_t* input_sizes,
                              size_t num_inputs, void* const* outputs, const size_t* output_sizes, size_t num_outputs,
                              void* stream, const char** error_message);

#ifdef __cplusplus
}
#endif

#endif /* RYFT_MI355X_H_ */
