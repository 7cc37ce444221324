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

#ifdef __cplusplus
}
#endif

#endif /* RYFT_MI355X_H_ */
