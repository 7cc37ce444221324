// Host-path check under ThreadSanitizer (built by the Makefile beside this file, run by tests/test_sanitize.py on the
// CPU): the plugin's C API driven from several threads at once on a compile-only client, no GPU —
//   * compiles of every program file named on the command line, on one shared client, from four threads;
//   * profiler sessions created, started, stopped, collected and destroyed meanwhile (every compile records its host
//     span into every started session);
//   * user events (PJRT_Event_Create / Set) with OnReady callbacks registered from three threads while a fourth sets
//     the events (half of them with an error) and two more await and poll them: each callback must run exactly once
//     and see its event's outcome.
// These are the plugin's shared-state surfaces (clients.rs:11-14 and events.rs:146-198 give ryft-pjrt's thread-safety
// contract). A data race or lock-order report from the sanitizer, or a wrong callback count, fails the run.
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>
#include <string>
#include <thread>
#include <vector>

#include "pjrt_c_api.h"

extern "C" const PJRT_Api* GetPjrtApi(void);

namespace {

const PJRT_Api* g_api = nullptr;

template <typename T>
T args() {
  T a;
  std::memset(&a, 0, sizeof a);
  a.struct_size = sizeof a;
  return a;
}

std::string message(PJRT_Error* e) {
  auto m = args<PJRT_Error_Message_Args>();
  m.error = e;
  g_api->PJRT_Error_Message(&m);
  return std::string(m.message, m.message_size);
}

int code_of(PJRT_Error* e) {
  auto c = args<PJRT_Error_GetCode_Args>();
  c.error = e;
  g_api->PJRT_Error_GetCode(&c);
  return (int)c.code;
}

void destroy(PJRT_Error* e) {
  auto d = args<PJRT_Error_Destroy_Args>();
  d.error = e;
  g_api->PJRT_Error_Destroy(&d);
}

[[noreturn]] void die(const std::string& what) {
  std::fprintf(stderr, "tsan_check: %s\n", what.c_str());
  std::exit(1);
}

void ok(PJRT_Error* e, const char* what) {
  if (!e) return;
  const std::string m = message(e);
  destroy(e);
  die(std::string(what) + ": " + m);
}

// ------------------------------------------------------------------------------------------------ compiles
void compile_worker(PJRT_Client* client, const std::vector<std::string>* programs, int rounds, std::atomic<long>* n) {
  for (int r = 0; r < rounds; ++r)
    for (const std::string& text : *programs) {
      PJRT_Program prog;
      std::memset(&prog, 0, sizeof prog);
      prog.struct_size = sizeof prog;
      prog.code = const_cast<char*>(text.data());
      prog.code_size = text.size();
      prog.format = "mlir";
      prog.format_size = 4;
      auto c = args<PJRT_Client_Compile_Args>();
      c.client = client;
      c.program = &prog;
      ok(g_api->PJRT_Client_Compile(&c), "compile");
      auto g = args<PJRT_LoadedExecutable_GetExecutable_Args>();
      g.loaded_executable = c.executable;
      ok(g_api->PJRT_LoadedExecutable_GetExecutable(&g), "get executable");
      auto no = args<PJRT_Executable_NumOutputs_Args>();
      no.executable = g.executable;
      ok(g_api->PJRT_Executable_NumOutputs(&no), "num outputs");
      auto de = args<PJRT_Executable_Destroy_Args>();
      de.executable = g.executable;
      ok(g_api->PJRT_Executable_Destroy(&de), "executable destroy");
      auto dl = args<PJRT_LoadedExecutable_Destroy_Args>();
      dl.executable = c.executable;
      ok(g_api->PJRT_LoadedExecutable_Destroy(&dl), "loaded executable destroy");
      n->fetch_add(1);
    }
}

// ------------------------------------------------------------------------------------------------ profiler
const PLUGIN_Profiler_Api* profiler_api() {
  for (const PJRT_Extension_Base* e = g_api->extension_start; e; e = e->next)
    if (e->extension_type == PJRT_Extension_Type_Profiler) return reinterpret_cast<const PJRT_Profiler_Extension*>(e)->profiler_api;
  die("no profiler extension");
}

void profiler_ok(const PLUGIN_Profiler_Api* p, PLUGIN_Profiler_Error* e, const char* what) {
  if (!e) return;
  PLUGIN_Profiler_Error_Message_Args m;
  std::memset(&m, 0, sizeof m);
  m.struct_size = sizeof m;
  m.error = e;
  p->PLUGIN_Profiler_Error_Message(&m);
  const std::string msg(m.message, m.message_size);
  PLUGIN_Profiler_Error_Destroy_Args d;
  std::memset(&d, 0, sizeof d);
  d.struct_size = sizeof d;
  d.error = e;
  p->PLUGIN_Profiler_Error_Destroy(&d);
  die(std::string(what) + ": " + msg);
}

// at least `sessions` sessions, and more until the compiles end
void profiler_worker(int sessions, const std::atomic<bool>* stop) {
  const PLUGIN_Profiler_Api* p = profiler_api();
  for (int s = 0; s < sessions || !stop->load(); ++s) {
    PLUGIN_Profiler_Create_Args c;
    std::memset(&c, 0, sizeof c);
    c.struct_size = sizeof c;
    profiler_ok(p, p->PLUGIN_Profiler_Create(&c), "profiler create");
    PLUGIN_Profiler_Start_Args st{sizeof(PLUGIN_Profiler_Start_Args), c.profiler};
    profiler_ok(p, p->PLUGIN_Profiler_Start(&st), "profiler start");
    std::this_thread::sleep_for(std::chrono::milliseconds(2));
    PLUGIN_Profiler_Stop_Args sp{sizeof(PLUGIN_Profiler_Stop_Args), c.profiler};
    profiler_ok(p, p->PLUGIN_Profiler_Stop(&sp), "profiler stop");
    PLUGIN_Profiler_CollectData_Args cd;
    std::memset(&cd, 0, sizeof cd);
    cd.struct_size = sizeof cd;
    cd.profiler = c.profiler;
    profiler_ok(p, p->PLUGIN_Profiler_CollectData(&cd), "profiler collect");
    if (!cd.buffer || cd.buffer_size_in_bytes == 0) die("profiler collected nothing");
    PLUGIN_Profiler_Destroy_Args d{sizeof(PLUGIN_Profiler_Destroy_Args), c.profiler};
    profiler_ok(p, p->PLUGIN_Profiler_Destroy(&d), "profiler destroy");
  }
}

// ------------------------------------------------------------------------------------------------ events
constexpr int kEvents = 200, kRegistrars = 3;

struct Seen {
  std::atomic<int> calls{0};
  std::atomic<int> errors{0};
};

void on_ready(PJRT_Error* e, void* user) {
  auto* s = static_cast<Seen*>(user);
  if (e) {
    if (code_of(e) != PJRT_Error_Code_ABORTED || message(e) != "event failed") die("callback saw the wrong error");
    s->errors.fetch_add(1);
    destroy(e);
  }
  s->calls.fetch_add(1);
}

void event_check() {
  std::vector<PJRT_Event*> ev(kEvents);
  for (auto& e : ev) {
    auto c = args<PJRT_Event_Create_Args>();
    ok(g_api->PJRT_Event_Create(&c), "event create");
    e = c.event;
  }
  std::vector<Seen> seen(kEvents * kRegistrars);
  std::vector<std::thread> th;
  for (int r = 0; r < kRegistrars; ++r)
    th.emplace_back([&, r] {
      for (int i = 0; i < kEvents; ++i) {
        auto o = args<PJRT_Event_OnReady_Args>();
        o.event = ev[i];
        o.callback = on_ready;
        o.user_arg = &seen[i * kRegistrars + r];
        ok(g_api->PJRT_Event_OnReady(&o), "on ready");
      }
    });
  th.emplace_back([&] {
    for (int i = 0; i < kEvents; ++i) {
      auto s = args<PJRT_Event_Set_Args>();
      s.event = ev[i];
      s.error_code = i % 2 ? PJRT_Error_Code_ABORTED : PJRT_Error_Code_OK;
      s.error_message = "event failed";
      s.error_message_size = std::strlen(s.error_message);
      ok(g_api->PJRT_Event_Set(&s), "event set");
    }
  });
  for (int w = 0; w < 2; ++w)
    th.emplace_back([&, w] {
      for (int k = 0; k < kEvents; ++k) {
        const int i = w ? kEvents - 1 - k : k;
        auto r = args<PJRT_Event_IsReady_Args>();
        r.event = ev[i];
        ok(g_api->PJRT_Event_IsReady(&r), "is ready");
        auto a = args<PJRT_Event_Await_Args>();
        a.event = ev[i];
        PJRT_Error* e = g_api->PJRT_Event_Await(&a);
        if ((e != nullptr) != (i % 2 == 1)) die("await saw the wrong outcome");
        if (e) destroy(e);
        auto er = args<PJRT_Event_Error_Args>();
        er.event = ev[i];
        e = g_api->PJRT_Event_Error(&er);
        if ((e != nullptr) != (i % 2 == 1)) die("event error saw the wrong outcome");
        if (e) destroy(e);
      }
    });
  for (auto& t : th) t.join();
  for (int i = 0; i < kEvents; ++i)
    for (int r = 0; r < kRegistrars; ++r) {
      const Seen& s = seen[i * kRegistrars + r];
      if (s.calls.load() != 1 || s.errors.load() != (i % 2)) die("OnReady callback count / outcome wrong");
    }
  for (auto& e : ev) {
    auto d = args<PJRT_Event_Destroy_Args>();
    d.event = e;
    ok(g_api->PJRT_Event_Destroy(&d), "event destroy");
  }
}

}  // namespace

int main(int argc, char** argv) {
  g_api = GetPjrtApi();
  std::vector<std::string> programs;
  for (int i = 1; i < argc; ++i) {
    std::ifstream f(argv[i], std::ios::binary);
    if (!f) die(std::string("cannot read ") + argv[i]);
    programs.emplace_back(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
  }
  if (programs.empty()) die("no program files");
  auto init = args<PJRT_Plugin_Initialize_Args>();
  ok(g_api->PJRT_Plugin_Initialize(&init), "initialize");

  PJRT_NamedValue opt;
  std::memset(&opt, 0, sizeof opt);
  opt.struct_size = sizeof opt;
  opt.name = "compile_only";
  opt.name_size = std::strlen(opt.name);
  opt.type = PJRT_NamedValue_kBool;
  opt.bool_value = true;
  opt.value_size = 1;
  auto cc = args<PJRT_Client_Create_Args>();
  cc.create_options = &opt;
  cc.num_options = 1;
  ok(g_api->PJRT_Client_Create(&cc), "client create");

  std::atomic<long> compiled{0};
  std::atomic<bool> stop{false};
  std::vector<std::thread> th;
  for (int w = 0; w < 4; ++w) th.emplace_back(compile_worker, cc.client, &programs, 30, &compiled);
  std::thread prof(profiler_worker, 20, &stop);
  event_check();
  for (auto& t : th) t.join();
  stop = true;
  prof.join();

  auto cd = args<PJRT_Client_Destroy_Args>();
  cd.client = cc.client;
  ok(g_api->PJRT_Client_Destroy(&cd), "client destroy");
  std::printf("tsan_check: %ld compiles on 4 threads beside profiler sessions, %d events x %d callbacks\n",
              compiled.load(), kEvents, kRegistrars);
  return 0;
}
