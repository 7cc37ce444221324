// Host-path check under AddressSanitizer and UndefinedBehaviorSanitizer (built by the Makefile beside this file,
// run by tests/test_sanitize.py on the CPU): every file named on the command line is fed to the plugin's compile path
// without a GPU — MLIR text (.mlir) and MLIR bytecode (.mlirbc) are parsed and planned, CompileOptionsProto bytes
// (.pb) decoded — and so is every truncation and bit-flipped copy the mutation schedule below derives from it.
// Rejections (the plugin's Status exceptions, which the C API turns into PJRT errors) are expected; a sanitizer
// report or any other exception ends the process with a failure.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

#include "ir.h"
#include "planner.h"
#include "runtime.h"

namespace ryft {
// the kernel library's launchers read the runtime's per-thread start event; nothing is launched here
hipEvent_t& pending_start() {
  static thread_local hipEvent_t e = nullptr;
  return e;
}
}  // namespace ryft

namespace {

struct Counts {
  long accepted = 0, rejected = 0;
};

enum class Kind { Text, Bytecode, Options };

const char* g_file = "";
const char* g_what = "";
size_t g_at = 0;

void feed(Kind kind, const std::string& bytes, Counts& n) {
  try {
    if (kind == Kind::Options) {
      ryft::CompileOptions o = ryft::decode_compile_options(bytes);
      (void)ryft::choose_device(o, 1);
    } else {
      ryft::Graph g = kind == Kind::Bytecode ? ryft::parse_mlir_bytecode(bytes, "main") : ryft::parse_mlir_text(bytes, "main");
      ryft::PlanOptions po;
      ryft::Plan p = ryft::build_plan(g, po);
      (void)p;
    }
    ++n.accepted;
  } catch (const ryft::Status&) {
    ++n.rejected;
  } catch (const std::exception& e) {
    // anything but a Status would escape the C API as an unexpected exception
    std::fprintf(stderr, "%s (%s at %zu, %zu bytes): unexpected exception: %s\n", g_file, g_what, g_at, bytes.size(),
                 e.what());
    std::exit(1);
  }
}

// Truncations at every length up to 64 bytes and at up to 96 evenly spaced lengths beyond; single-bit flips at up
// to 192 evenly spaced positions (bit position varying with the byte), and the bytes there forced to 0x00 and 0xFF.
void mutate(Kind kind, const std::string& s, Counts& n) {
  const size_t len = s.size();
  g_what = "truncation";
  for (size_t l = 0; l < len && l <= 64; ++l) feed(kind, s.substr(0, g_at = l), n);
  const size_t tstep = len > 64 ? (len - 64) / 96 + 1 : 1;
  for (size_t l = 65; l < len; l += tstep) feed(kind, s.substr(0, g_at = l), n);
  if (len == 0) return;
  const size_t fstep = len / 192 + 1;
  for (size_t i = 0; i < len; i += fstep) {
    std::string t = s;
    g_at = i;
    t[i] = (char)(t[i] ^ (1u << (i % 8)));
    g_what = "bit flip";
    feed(kind, t, n);
    t[i] = 0;
    g_what = "zero byte";
    feed(kind, t, n);
    t[i] = (char)0xFF;
    g_what = "0xff byte";
    feed(kind, t, n);
  }
}

}  // namespace

int main(int argc, char** argv) {
  Counts plain, mutated;
  int files = 0;
  for (int i = 1; i < argc; ++i) {
    const std::string path = argv[i];
    std::ifstream f(path, std::ios::binary);
    if (!f) {
      std::fprintf(stderr, "cannot read %s\n", path.c_str());
      return 2;
    }
    const std::string bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    auto ends = [&](const char* suf) {
      const size_t k = std::strlen(suf);
      return path.size() >= k && path.compare(path.size() - k, k, suf) == 0;
    };
    const Kind kind = ends(".mlirbc") ? Kind::Bytecode : ends(".pb") ? Kind::Options : Kind::Text;
    ++files;
    g_file = argv[i];
    g_what = "as it is";
    const long before = plain.rejected;
    feed(kind, bytes, plain);
    if (kind != Kind::Options && plain.rejected != before)
      std::fprintf(stderr, "note: %s is rejected as it is\n", path.c_str());
    mutate(kind, bytes, mutated);
  }
  std::printf("frontend_check: %d files (%ld accepted, %ld rejected as they are); %ld mutated inputs (%ld accepted, "
              "%ld rejected)\n",
              files, plain.accepted, plain.rejected, mutated.accepted + mutated.rejected, mutated.accepted,
              mutated.rejected);
  return 0;
}
