/* GetPjrtApi, like crates/ryft-xla-sys/pjrt_plugin_version_script.lds, plus the allocation-free execute entry point
   (no counterpart in the reference). */
VERS_1.0 {
  global:
    GetPjrtApi;
    RyftMi355x_ExecuteNoAlloc;
  local:
    *;
};
