/* The plugin exports exactly one symbol, like crates/ryft-xla-sys/pjrt_plugin_version_script.lds. */
VERS_1.0 {
  global:
    GetPjrtApi;
  local:
    *;
};
