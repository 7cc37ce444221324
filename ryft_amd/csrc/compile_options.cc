// CompileOptionsProto decoding (the bytes ryft-pjrt passes to PJRT_Client_Compile).
//
// Message layout per crates/ryft-xla-sys/src/protos.rs:3298-3346 (CompilationOptions) and :2391-2530
// (ExecutableCompilationOptions), proto3 wire format. Fields the plugin acts on are decoded; the rest are skipped by
// wire type so that options written by newer producers still compile.
#include <string>

#include "runtime.h"

namespace ryft {
namespace {

// A protobuf wire-format reader over one message's bytes.
struct ProtoReader {
  const uint8_t* p;
  const uint8_t* end;
  const char* what;

  bool done() const { return p >= end; }
  [[noreturn]] void bad(const std::string& why) const {
    invalid(std::string("malformed compile options (") + what + "): " + why);
  }
  uint64_t varint() {
    uint64_t v = 0;
    for (int shift = 0; shift < 64; shift += 7) {
      if (p >= end) bad("truncated varint");
      const uint8_t b = *p++;
      v |= (uint64_t)(b & 0x7f) << shift;
      if (!(b & 0x80)) return v;
    }
    bad("varint longer than 10 bytes");
  }
  // a length-delimited field's bytes
  ProtoReader sub(const char* name) {
    const uint64_t n = varint();
    if (n > (uint64_t)(end - p)) bad(std::string("field ") + name + " runs past the end");
    ProtoReader r{p, p + n, name};
    p += n;
    return r;
  }
  void skip(int wire) {
    switch (wire) {
      case 0: varint(); return;
      case 1: if (end - p < 8) bad("truncated fixed64"); p += 8; return;
      case 2: sub("skipped field"); return;
      case 5: if (end - p < 4) bad("truncated fixed32"); p += 4; return;
      default: bad("unsupported wire type " + std::to_string(wire));
    }
  }
  void expect(int wire, int want, const char* name) {
    if (wire != want) bad(std::string("field ") + name + " has wire type " + std::to_string(wire));
  }
};

// xla.DeviceAssignmentProto: replica_count (1), computation_count (2), computation_devices (3, repeated
// {replica_device_ids (1, repeated int64, packed or not)}); device ids in replica-major order per computation.
void decode_device_assignment(ProtoReader r, CompileOptions* o) {
  int64_t replicas = 0, computations = 0;
  std::vector<int64_t> ids;
  while (!r.done()) {
    const uint64_t key = r.varint();
    const int num = (int)(key >> 3), wire = (int)(key & 7);
    if (num == 1) { r.expect(wire, 0, "replica_count"); replicas = (int64_t)r.varint(); }
    else if (num == 2) { r.expect(wire, 0, "computation_count"); computations = (int64_t)r.varint(); }
    else if (num == 3) {
      r.expect(wire, 2, "computation_devices");
      ProtoReader cd = r.sub("computation_devices");
      while (!cd.done()) {
        const uint64_t k = cd.varint();
        if ((k >> 3) != 1) { cd.skip((int)(k & 7)); continue; }
        if ((k & 7) == 0) {
          ids.push_back((int64_t)cd.varint());
        } else if ((k & 7) == 2) {
          ProtoReader packed = cd.sub("replica_device_ids");
          while (!packed.done()) ids.push_back((int64_t)packed.varint());
        } else {
          cd.bad("replica_device_ids has wire type " + std::to_string(k & 7));
        }
      }
    } else {
      r.skip(wire);
    }
  }
  if (replicas * computations != (int64_t)ids.size())
    invalid("compile options: the device assignment names " + std::to_string(ids.size()) + " device(s) for " +
            std::to_string(replicas) + " replica(s) × " + std::to_string(computations) + " computation(s)");
  o->assignment_replicas = replicas;
  o->assignment_computations = computations;
  o->assignment_ids = ids;
}

void decode_build_options(ProtoReader r, CompileOptions* o) {
  while (!r.done()) {
    const uint64_t key = r.varint();
    const int num = (int)(key >> 3), wire = (int)(key & 7);
    switch (num) {
      case 1: r.expect(wire, 0, "device_ordinal"); o->device_ordinal = (int64_t)r.varint(); break;
      case 4: r.expect(wire, 0, "replica_count"); o->replica_count = (int64_t)r.varint(); break;
      case 5: r.expect(wire, 0, "partition_count"); o->partition_count = (int64_t)r.varint(); break;
      case 6: r.expect(wire, 0, "use_spmd_partitioning"); o->use_spmd_partitioning = r.varint() != 0; break;
      case 9: r.expect(wire, 2, "device_assignment"); decode_device_assignment(r.sub("device_assignment"), o); break;
      default: r.skip(wire); break;
    }
  }
}

}  // namespace

CompileOptions decode_compile_options(const std::string& bytes) {
  CompileOptions o;
  ProtoReader r{(const uint8_t*)bytes.data(), (const uint8_t*)bytes.data() + bytes.size(), "CompileOptionsProto"};
  while (!r.done()) {
    const uint64_t key = r.varint();
    const int num = (int)(key >> 3), wire = (int)(key & 7);
    switch (num) {
      case 2: r.expect(wire, 0, "parameter_is_tupled_arguments"); o.tupled_arguments = r.varint() != 0; break;
      case 3:
        r.expect(wire, 2, "executable_build_options");
        decode_build_options(r.sub("executable_build_options"), &o);
        break;
      case 4: r.expect(wire, 0, "compile_portable_executable"); o.portable = r.varint() != 0; break;
      case 10: r.expect(wire, 0, "matrix_unit_operand_precision"); o.precision = (int)r.varint(); break;
      default: r.skip(wire); break;
    }
  }
  // what one executable of this plugin can be: one replica, one partition, untupled parameters
  if (o.tupled_arguments) unimplemented("compile options: tupled parameters (parameter_is_tupled_arguments) are not supported");
  if (o.replica_count > 1 || o.partition_count > 1)
    unimplemented("compile options: " + std::to_string(o.replica_count) + " replica(s) × " +
                  std::to_string(o.partition_count) + " partition(s) requested; this plugin compiles for one device "
                  "(one replica, one partition)");
  if (o.replica_count < 0 || o.partition_count < 0) invalid("compile options: negative replica or partition count");
  if (!o.assignment_ids.empty() && o.assignment_ids.size() != 1)
    unimplemented("compile options: a device assignment over " + std::to_string(o.assignment_ids.size()) +
                  " devices; this plugin compiles for one device");
  if (o.precision < 0 || o.precision > 2)
    invalid("compile options: unknown matrix_unit_operand_precision " + std::to_string(o.precision));
  return o;
}

int choose_device(const CompileOptions& o, size_t num_devices) {
  int64_t dev = 0;
  if (!o.assignment_ids.empty()) dev = o.assignment_ids[0];
  if (o.device_ordinal >= 0) {
    if (!o.assignment_ids.empty() && o.assignment_ids[0] != o.device_ordinal)
      invalid("compile options: device_ordinal " + std::to_string(o.device_ordinal) +
              " disagrees with the device assignment (device " + std::to_string(o.assignment_ids[0]) + ")");
    dev = o.device_ordinal;
  } else if (o.device_ordinal < -1) {
    invalid("compile options: device_ordinal " + std::to_string(o.device_ordinal));
  }
  if (num_devices && (dev < 0 || dev >= (int64_t)num_devices))
    invalid("compile options name device " + std::to_string(dev) + " but the client has " +
            std::to_string(num_devices) + " device(s)");
  return (int)dev;
}

}  // namespace ryft
