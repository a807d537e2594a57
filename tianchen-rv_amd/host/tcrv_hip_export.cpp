// tcrv_hip_export -- writes the exported C++ of a set of selected variants:
// for each manifest line, the tcrv_emitc_<kernel>_<variant> function
// libtcrv_hip_route's tcrv_hip_export_function renders, into one translation
// unit plus a header of their prototypes.  The generated unit is plain C++
// over tcrv_hip.h (compile it with g++ and link libtcrv_hip).
//
//   tcrv_hip_export MANIFEST OUT.cpp OUT.h
//
// Manifest: one variant per line, `#` starts a comment:
//   <op identity> <kernel symbol> <variant symbol> [key=value ...]
// with the op facts the emitted C bakes in as keys:
//   kind=add|sub|mul, elem=i8|u8|i16|u16|i32|u32|i64|f32|f64  (tcrv_rvv.binary)
//   activation_cols=<n>                                    (the GEMM tile)
// Exit status 0, or 1 with a message naming the manifest line.
#include <cctype>
#include <cstdint>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "tcrv_hip_route.h"

namespace {

const std::map<std::string, int64_t> kKinds = {
    {"add", TCRV_HIP_BINARY_ADD}, {"sub", TCRV_HIP_BINARY_SUB}, {"mul", TCRV_HIP_BINARY_MUL}};
const std::map<std::string, int64_t> kElems = {
    {"i8", TCRV_HIP_ELEM_I8},   {"u8", TCRV_HIP_ELEM_U8},   {"i16", TCRV_HIP_ELEM_I16},
    {"u16", TCRV_HIP_ELEM_U16}, {"i32", TCRV_HIP_ELEM_I32}, {"u32", TCRV_HIP_ELEM_U32},
    {"i64", TCRV_HIP_ELEM_I64}, {"f32", TCRV_HIP_ELEM_F32}, {"f64", TCRV_HIP_ELEM_F64}};

struct Variant {
  std::string op, kernel, variant;
  std::vector<int64_t> attrs;  // {kind, elem} or {activation_cols}
};

// Parses one manifest line; false (with `err`) on a malformed one.  Blank and
// comment-only lines give an empty op.
bool parseLine(const std::string &raw, Variant &v, std::string &err) {
  std::string line = raw.substr(0, raw.find('#'));
  std::istringstream in(line);
  if (!(in >> v.op))
    return true;
  if (!(in >> v.kernel >> v.variant)) {
    err = "expected <op> <kernel> <variant>";
    return false;
  }
  int64_t kind = -1, elem = -1, cols = -1;
  std::string kv;
  while (in >> kv) {
    const size_t eq = kv.find('=');
    if (eq == std::string::npos) {
      err = "attribute without '=': " + kv;
      return false;
    }
    const std::string key = kv.substr(0, eq), val = kv.substr(eq + 1);
    if (key == "kind" && kKinds.count(val)) {
      kind = kKinds.at(val);
    } else if (key == "elem" && kElems.count(val)) {
      elem = kElems.at(val);
    } else if (key == "activation_cols") {
      char *end = nullptr;
      cols = std::strtoll(val.c_str(), &end, 10);
      if (!end || *end != '\0' || cols < 1) {
        err = "activation_cols is not a positive integer: " + val;
        return false;
      }
    } else {
      err = "unknown attribute: " + kv;
      return false;
    }
  }
  if (kind >= 0 || elem >= 0)
    v.attrs = {kind, elem};
  else if (cols >= 0)
    v.attrs = {cols};
  return true;
}

bool render(const Variant &v, int form, std::string &out, std::string &err) {
  size_t need = 0;
  const int64_t *attrs = v.attrs.empty() ? nullptr : v.attrs.data();
  int st = tcrv_hip_export_function(v.op.c_str(), v.kernel.c_str(), v.variant.c_str(), attrs,
                                    v.attrs.size(), form, nullptr, 0, &need);
  if (st == TCRV_HIP_OK) {
    std::vector<char> buf(need);
    st = tcrv_hip_export_function(v.op.c_str(), v.kernel.c_str(), v.variant.c_str(), attrs,
                                  v.attrs.size(), form, buf.data(), buf.size(), nullptr);
    out += buf.data();
  }
  if (st != TCRV_HIP_OK)
    err = std::string(st == TCRV_HIP_ERR_UNSUPPORTED ? "no route row for " : "bad attributes for ") +
          v.op;
  return st == TCRV_HIP_OK;
}

std::string guardOf(const std::string &path) {
  std::string base = path.substr(path.find_last_of('/') + 1), g;
  for (char c : base)
    g += std::isalnum(static_cast<unsigned char>(c)) ? static_cast<char>(std::toupper(c)) : '_';
  return g + "_";
}

}  // namespace

int main(int argc, char **argv) {
  if (argc != 4) {
    std::fprintf(stderr, "usage: %s MANIFEST OUT.cpp OUT.h\n", argv[0]);
    return 1;
  }
  std::ifstream manifest(argv[1]);
  if (!manifest) {
    std::fprintf(stderr, "%s: cannot read\n", argv[1]);
    return 1;
  }
  const std::string hdrPath = argv[3];
  const std::string hdrName = hdrPath.substr(hdrPath.find_last_of('/') + 1);
  std::string defs, decls;
  std::string raw, err;
  for (int lineNo = 1; std::getline(manifest, raw); ++lineNo) {
    Variant v;
    if (!parseLine(raw, v, err) ||
        (!v.op.empty() && (!render(v, TCRV_HIP_EXPORT_DEFINITION, defs, err) ||
                           !render(v, TCRV_HIP_EXPORT_DECLARATION, decls, err)))) {
      std::fprintf(stderr, "%s:%d: %s\n", argv[1], lineNo, err.c_str());
      return 1;
    }
    if (!v.op.empty())
      defs += "\n";
  }
  const std::string guard = guardOf(hdrPath);
  std::ofstream h(hdrPath), c(argv[2]);
  h << "// Prototypes of the exported variants (generated by tcrv_hip_export).\n"
    << "#ifndef " << guard << "\n#define " << guard << "\n\n#include <stddef.h>\n#include "
    << "<stdint.h>\n\n" << decls << "\n#endif  // " << guard << "\n";
  c << tcrv_hip_export_prologue() << "#include \"" << hdrName << "\"\n\n" << defs;
  if (!h || !c) {
    std::fprintf(stderr, "cannot write %s or %s\n", argv[2], argv[3]);
    return 1;
  }
  return 0;
}
