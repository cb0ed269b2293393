// abi.cpp -- library-wide C ABI: version, the materialization contract of the
// reference (block-size JSON -> variant names, variant name -> tile values)
// and the by-name dispatcher a backend seam calls.
//
// Reference behaviour mirrored here:
//   - block-size JSON (lib/pipeline/src/loom_materialization_pipeline.cpp:
//     81-192): a top-level object; each key names a function and maps to a
//     binding object {"sym": int, ...}, a non-empty array of such objects, or
//     null (UNSAT: the function is skipped); "__loom_candidate_order__" maps
//     to an array of strings; symbol values must be integers; "ALL" expands
//     to every function that has no binding of its own (:251-270);
//   - variant names (lib/passes/loom-opt/src/materialize.cpp:39-53,253-262):
//     <function> + "__<sym><value>" for every bound symbol in sorted symbol
//     order, with "__combo<i>" appended while a name is already taken;
//   - error reporting as (code, message), the pipeline's "(error, result)"
//     convention (lib/pipeline/__init__.py:97-98).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cctype>
#include <cerrno>
#include <cstdlib>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <utility>
#include <vector>

#include "../../include/loom_hip.h"

#define LOOM_HIP_VERSION_STRING "loom_hip 0.2.0 gfx950"

namespace {

int fail(char* err, size_t errlen, int code, const char* fmt, ...) {
  if (err && errlen) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
  }
  return code;
}

// ---------------------------------------------------------------------------
// Minimal JSON reader: objects (key order kept), arrays, strings, numbers
// (integer-valued or not), true/false/null.
// ---------------------------------------------------------------------------
struct JVal {
  enum Kind { Null, Bool, Int, Real, Str, Arr, Obj } kind = Null;
  bool b = false;
  long long i = 0;
  std::string s;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
};

struct JParser {
  const char* p;
  const char* end;
  std::string err;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool bad(const char* what) {
    if (err.empty()) err = what;
    return false;
  }
  bool lit(const char* w) {
    const size_t n = strlen(w);
    if ((size_t)(end - p) < n || strncmp(p, w, n) != 0) return false;
    p += n;
    return true;
  }
  bool str(std::string& out) {
    if (p >= end || *p != '"') return bad("expected a string");
    ++p;
    out.clear();
    while (p < end && *p != '"') {
      char c = *p++;
      if (c == '\\') {
        if (p >= end) return bad("unterminated escape");
        const char e = *p++;
        switch (e) {
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          case '/': out += '/'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {
            if (end - p < 4) return bad("short \\u escape");
            unsigned v = 0;
            for (int k = 0; k < 4; ++k) {
              const char h = *p++;
              v <<= 4;
              if (h >= '0' && h <= '9') v |= h - '0';
              else if (h >= 'a' && h <= 'f') v |= h - 'a' + 10;
              else if (h >= 'A' && h <= 'F') v |= h - 'A' + 10;
              else return bad("bad \\u escape");
            }
            if (v < 0x80) {
              out += (char)v;
            } else if (v < 0x800) {
              out += (char)(0xC0 | (v >> 6));
              out += (char)(0x80 | (v & 0x3F));
            } else {
              out += (char)(0xE0 | (v >> 12));
              out += (char)(0x80 | ((v >> 6) & 0x3F));
              out += (char)(0x80 | (v & 0x3F));
            }
            break;
          }
          default: return bad("bad escape");
        }
      } else {
        out += c;
      }
    }
    if (p >= end) return bad("unterminated string");
    ++p;
    return true;
  }
  bool num(JVal& v) {
    const char* s = p;
    if (p < end && *p == '-') ++p;
    if (p >= end || !isdigit((unsigned char)*p)) return bad("bad number");
    while (p < end && isdigit((unsigned char)*p)) ++p;
    bool real = false;
    if (p < end && *p == '.') {
      real = true;
      ++p;
      if (p >= end || !isdigit((unsigned char)*p)) return bad("bad number");
      while (p < end && isdigit((unsigned char)*p)) ++p;
    }
    if (p < end && (*p == 'e' || *p == 'E')) {
      real = true;
      ++p;
      if (p < end && (*p == '+' || *p == '-')) ++p;
      if (p >= end || !isdigit((unsigned char)*p)) return bad("bad number");
      while (p < end && isdigit((unsigned char)*p)) ++p;
    }
    const std::string t(s, p);
    if (!real) {
      errno = 0;
      char* e = nullptr;
      const long long x = strtoll(t.c_str(), &e, 10);
      if (errno == ERANGE) return bad("integer out of range");
      v.kind = JVal::Int;
      v.i = x;
      return true;
    }
    // a real number that happens to be integral (e.g. 64.0) is still an
    // integer value, as llvm::json::Value::getAsInteger accepts it
    const double d = strtod(t.c_str(), nullptr);
    // range first: converting a double outside long long's range (or inf)
    // to long long is undefined
    if (d > -9.2e18 && d < 9.2e18 && d == (double)(long long)d) {
      v.kind = JVal::Int;
      v.i = (long long)d;
    } else {
      v.kind = JVal::Real;
    }
    return true;
  }
  bool value(JVal& v, int depth) {
    if (depth > 64) return bad("nesting too deep");
    ws();
    if (p >= end) return bad("unexpected end of input");
    const char c = *p;
    if (c == '{') {
      ++p;
      v.kind = JVal::Obj;
      ws();
      if (p < end && *p == '}') {
        ++p;
        return true;
      }
      for (;;) {
        ws();
        std::string k;
        if (!str(k)) return false;
        ws();
        if (p >= end || *p != ':') return bad("expected ':'");
        ++p;
        JVal child;
        if (!value(child, depth + 1)) return false;
        v.obj.emplace_back(std::move(k), std::move(child));
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == '}') {
          ++p;
          return true;
        }
        return bad("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p;
      v.kind = JVal::Arr;
      ws();
      if (p < end && *p == ']') {
        ++p;
        return true;
      }
      for (;;) {
        JVal child;
        if (!value(child, depth + 1)) return false;
        v.arr.push_back(std::move(child));
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == ']') {
          ++p;
          return true;
        }
        return bad("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = JVal::Str;
      return str(v.s);
    }
    if (lit("true")) {
      v.kind = JVal::Bool;
      v.b = true;
      return true;
    }
    if (lit("false")) {
      v.kind = JVal::Bool;
      return true;
    }
    if (lit("null")) {
      v.kind = JVal::Null;
      return true;
    }
    return num(v);
  }
};

bool parse_json(const std::string& text, JVal& root, std::string& err) {
  JParser jp{text.data(), text.data() + text.size(), {}};
  if (!jp.value(root, 0)) {
    err = jp.err;
    return false;
  }
  jp.ws();
  if (jp.p != jp.end) {
    err = "trailing characters after the JSON value";
    return false;
  }
  return true;
}

// ---------------------------------------------------------------------------
// Block-size map (function -> bindings), as the materialization pipeline
// builds it.
// ---------------------------------------------------------------------------
typedef std::map<std::string, long long> Binding;  // sorted by symbol name

struct BlockSizes {
  std::vector<std::pair<std::string, std::vector<Binding>>> funcs;  // key order
  std::vector<std::string> candidate_order;
  bool has_all = false;
  std::vector<Binding> all;
};

bool parse_symbol_map(const std::string& fkey, const JVal& obj, Binding& out, std::string& err) {
  for (const auto& kv : obj.obj) {
    if (kv.second.kind != JVal::Int) {
      err = "Value for symbol '" + kv.first + "' in '" + fkey + "' must be an integer";
      return false;
    }
    out[kv.first] = kv.second.i;
  }
  return true;
}

bool parse_binding_list(const std::string& fkey, const JVal& v, std::vector<Binding>& out,
                        std::string& err) {
  if (v.kind == JVal::Obj) {
    Binding b;
    if (!parse_symbol_map(fkey, v, b, err)) return false;
    out.push_back(std::move(b));
    return true;
  }
  if (v.kind == JVal::Arr) {
    if (v.arr.empty()) {
      err = "Value for key '" + fkey + "' must not be an empty array";
      return false;
    }
    for (size_t i = 0; i < v.arr.size(); ++i) {
      if (v.arr[i].kind != JVal::Obj) {
        err = "Value for key '" + fkey + "' at index " + std::to_string(i) +
              " must be a JSON object";
        return false;
      }
      Binding b;
      if (!parse_symbol_map(fkey, v.arr[i], b, err)) return false;
      out.push_back(std::move(b));
    }
    return true;
  }
  err = "Value for key '" + fkey + "' must be a JSON object, array of objects, or null";
  return false;
}

bool parse_block_sizes(const std::string& text, BlockSizes& bs, std::string& err) {
  if (text.empty()) return true;  // the reference then uses its placeholder solver
  JVal root;
  std::string perr;
  if (!parse_json(text, root, perr)) {
    err = "Failed to parse block_sizes_json: " + perr;
    return false;
  }
  if (root.kind != JVal::Obj) {
    err = "block_sizes_json must be a JSON object at the top level";
    return false;
  }
  for (const auto& kv : root.obj) {
    const std::string& fkey = kv.first;
    if (fkey == "__loom_candidate_order__") {
      if (kv.second.kind != JVal::Arr) {
        err = "Value for '__loom_candidate_order__' must be an array";
        return false;
      }
      for (const auto& n : kv.second.arr) {
        if (n.kind != JVal::Str) {
          err = "Entries in '__loom_candidate_order__' must be strings";
          return false;
        }
        bs.candidate_order.push_back(n.s);
      }
      continue;
    }
    if (kv.second.kind == JVal::Null) continue;  // UNSAT: no variant emitted
    std::vector<Binding> bl;
    if (!parse_binding_list(fkey, kv.second, bl, err)) return false;
    if (fkey == "ALL") {
      bs.has_all = true;
      bs.all = std::move(bl);
      continue;
    }
    bool replaced = false;
    for (auto& f : bs.funcs)
      if (f.first == fkey) {
        f.second = bl;
        replaced = true;
      }
    if (!replaced) bs.funcs.emplace_back(fkey, std::move(bl));
  }
  return true;
}

std::string suffix_of(const Binding& b) {
  std::string s;
  for (const auto& kv : b) s += "__" + kv.first + std::to_string(kv.second);
  return s;
}

// ---------------------------------------------------------------------------
// Tile symbols the kernels know, and variant-name parsing
// ---------------------------------------------------------------------------
const char* const kTileNames[LOOM_HIP_NTILES] = {"tile_b", "tile_m", "tile_n", "tile_k",
                                                 "tile_s", "tile_h", "tile_c"};

int tile_index(const std::string& sym) {
  for (int i = 0; i < LOOM_HIP_NTILES; ++i)
    if (sym == kTileNames[i]) return i;
  return -1;
}

const char* const kFunctions[] = {"matmul", "batch_matmul", "split_k_matmul_gather",
                                  "attention", "flash_decode",
                                  "helion_mamba2_chunk_scan_kernel"};

bool known_function(const std::string& f) {
  for (const char* k : kFunctions)
    if (f == k) return true;
  return false;
}

// "<func>[__<mapping>...]__tile_k64__tile_m128[__comboN]" -> func, tiles.
// Tokens are the "__"-separated pieces after the function name; a token that
// starts with "tile_" and ends in digits binds that symbol, others (mapping
// variants, combo indices) are ignored.
int parse_variant(const std::string& name, std::string& func, int64_t* tiles,
                  std::string& err) {
  for (int i = 0; i < LOOM_HIP_NTILES; ++i) tiles[i] = -1;
  const size_t first = name.find("__");
  func = name.substr(0, first);
  if (func.empty()) {
    err = "variant name '" + name + "' has no function name";
    return LOOM_HIP_EINVAL;
  }
  size_t pos = first;
  while (pos != std::string::npos) {
    pos += 2;
    const size_t next = name.find("__", pos);
    const std::string tok = name.substr(pos, next == std::string::npos ? std::string::npos
                                                                         : next - pos);
    pos = next;
    if (tok.compare(0, 5, "tile_") != 0) continue;
    size_t d = tok.size();
    while (d > 0 && isdigit((unsigned char)tok[d - 1])) --d;
    if (d == tok.size()) {
      err = "variant token '" + tok + "' carries no value";
      return LOOM_HIP_EINVAL;
    }
    const std::string sym = tok.substr(0, d);
    const int ti = tile_index(sym);
    if (ti < 0) {
      err = "variant token '" + tok + "' names an unknown block-size symbol";
      return LOOM_HIP_EINVAL;
    }
    if (tok.size() - d > 12) {
      err = "variant token '" + tok + "' value out of range";
      return LOOM_HIP_EINVAL;
    }
    tiles[ti] = atoll(tok.c_str() + d);
  }
  return LOOM_HIP_OK;
}

// loom.sym symbols of each example function in order of first appearance
// (examples/*/IR/00_from_helion_frontend.mlir), which is the order the
// placeholder solver zips its candidate tuple with.
const std::vector<std::string>* known_symbols(const std::string& f) {
  static const std::map<std::string, std::vector<std::string>> table = {
      {"matmul", {"tile_m", "tile_n", "tile_k"}},
      {"batch_matmul", {"tile_b", "tile_m", "tile_n", "tile_k"}},
      {"split_k_matmul_gather", {"tile_m", "tile_n", "tile_k"}},
      {"attention", {"tile_b", "tile_m", "tile_n"}},
      {"flash_decode", {"tile_b", "tile_s", "tile_n"}},
      {"helion_mamba2_chunk_scan_kernel",
       {"tile_m", "tile_n", "tile_k", "tile_c", "tile_b", "tile_h"}},
  };
  auto it = table.find(f);
  return it == table.end() ? nullptr : &it->second;
}

// Placeholder solver of lib/passes/loom-opt/src/materialize.cpp:56-65: one
// candidate, {64,64,512} for three symbols, {64,32,64,8,1,4} for six, else 64
// for every symbol.
Binding placeholder_binding(const std::vector<std::string>& syms) {
  std::vector<long long> vals(syms.size(), 64);
  if (syms.size() == 3) vals = {64, 64, 512};
  if (syms.size() == 6) vals = {64, 32, 64, 8, 1, 4};
  Binding b;
  for (size_t i = 0; i < syms.size(); ++i) b[syms[i]] = vals[i];
  return b;
}

int need_tiles(const std::string& func, const int64_t* tiles, std::initializer_list<int> which,
               char* err, size_t errlen) {
  for (int i : which)
    if (tiles[i] < 0)
      return fail(err, errlen, LOOM_HIP_EINVAL, "dispatch: variant of %s lacks %s", func.c_str(),
                  kTileNames[i]);
  return LOOM_HIP_OK;
}

// ---------------------------------------------------------------------------
// gfx950 block-size constraint scopes, in the reference's constraint JSON
// grammar (lib/passes/lcs/inc/expr.h:17-25, constraint_expr.h:13-22):
//   Expr        {"Const": v} {"Sym": s} {"Add"|"Sub"|"Mul"|"Div"|"Min"|"Max": [a, b]}
//   Constraint  {"And"|"Or": [...]} {"Not": c} {"Eq"|"Le"|"Lt"|"Ge"|"Gt": [a, b]}
//               {"InRange": {"x", "lo", "hi"}} {"Divisible": {"x", "by"}}
// ---------------------------------------------------------------------------
std::string jc(long long v) { return "{\"Const\":" + std::to_string(v) + "}"; }
std::string js(const char* s) { return std::string("{\"Sym\":\"") + s + "\"}"; }
std::string jop(const char* op, const std::string& a, const std::string& b) {
  return std::string("{\"") + op + "\":[" + a + "," + b + "]}";
}
std::string jlist(const char* op, const std::vector<std::string>& xs) {
  std::string o = std::string("{\"") + op + "\":[";
  for (size_t i = 0; i < xs.size(); ++i) o += (i ? "," : "") + xs[i];
  return o + "]}";
}
std::string jrange(const char* sym, long long lo, long long hi) {
  return std::string("{\"InRange\":{\"x\":") + js(sym) + ",\"lo\":" + jc(lo) + ",\"hi\":" + jc(hi) + "}}";
}
std::string jdivisible(const char* sym, long long by) {
  return std::string("{\"Divisible\":{\"x\":") + js(sym) + ",\"by\":" + jc(by) + "}}";
}
std::string jsym(const char* name, long long ub, long long align) {
  return std::string("\"") + name + "\":{\"type\":\"int\",\"natural_ub\":" + std::to_string(ub) +
         ",\"alignment\":" + std::to_string(align) + "}";
}

constexpr long long kLdsBytes = 160 * 1024;   // LDS per workgroup on gfx950
constexpr long long kTileAlign = 16;          // MFMA tile edge (16x16x32)

struct Scope {
  std::vector<std::string> symbols, footprint, hard, temp_iter;
  std::string seq_iter;
};

int build_scope(const std::string& f, const int64_t* d, int nd, Scope& sc, std::string& err) {
  auto need = [&](int n) {
    if (nd != n) {
      err = "constraint_scope: " + f + " takes " + std::to_string(n) + " extents";
      return false;
    }
    for (int i = 0; i < n; ++i)
      if (d[i] <= 0) {
        err = "constraint_scope: extents must be positive";
        return false;
      }
    return true;
  };
  // Every symbol lies in [1, natural_ub] (the extent of the loop it tiles,
  // staged_etg_builder.cpp:1420-1430).  A tiled axis takes any multiple of
  // kTileAlign up to its extent, or the extent itself: the gfx950 analogue of
  // the reference's 32-alignment of inner tile dimensions
  // (hw_alignment.cpp:16).  It runs on the smallest built workgroup tile
  // covering it, or the largest built one above them all (loom_fit_tile in
  // csrc/common.h); no kernel's result depends on that choice.
  auto ub = [&](const char* sym, long long extent) { sc.hard.push_back(jrange(sym, 1, extent)); };
  auto tiled = [&](const char* sym, long long extent) {
    ub(sym, extent);
    sc.hard.push_back(jlist("Or", {jdivisible(sym, kTileAlign), jop("Eq", js(sym), jc(extent))}));
  };
  // GEMM workgroup tiles are square (64, 128 or 256); the A and B stage
  // rings hold at most 64 KB each (the 256 tile's four 16 KB stages; the
  // smaller tiles' rings are half that), the bound given here
  auto gemm_tiles = [&](long long M, long long N) {
    sc.symbols.push_back(jsym("tile_m", M, kTileAlign));
    sc.symbols.push_back(jsym("tile_n", N, kTileAlign));
    tiled("tile_m", M);
    tiled("tile_n", N);
    sc.footprint.push_back(jc(64 * 1024));
    sc.footprint.push_back(jc(64 * 1024));
    sc.hard.push_back(jop("Le", jop("Add", sc.footprint[0], sc.footprint[1]), jc(kLdsBytes)));
    sc.temp_iter.push_back(jop("Div", jc(M), js("tile_m")));
    sc.temp_iter.push_back(jop("Div", jc(N), js("tile_n")));
  };
  if (f == "matmul") {
    if (!need(3)) return LOOM_HIP_EINVAL;
    gemm_tiles(d[0], d[1]);
    sc.symbols.push_back(jsym("tile_k", d[2], 1));
    ub("tile_k", d[2]);
    sc.seq_iter = jop("Div", jc(d[2]), js("tile_k"));
  } else if (f == "batch_matmul") {
    if (!need(4)) return LOOM_HIP_EINVAL;
    sc.symbols.push_back(jsym("tile_b", d[0], 1));
    ub("tile_b", d[0]);
    gemm_tiles(d[1], d[2]);
    sc.symbols.push_back(jsym("tile_k", d[3], 1));
    ub("tile_k", d[3]);
    sc.temp_iter.insert(sc.temp_iter.begin(), jop("Div", jc(d[0]), js("tile_b")));
    sc.seq_iter = jop("Div", jc(d[3]), js("tile_k"));
  } else if (f == "split_k_matmul_gather") {
    if (!need(3)) return LOOM_HIP_EINVAL;
    gemm_tiles(d[0], d[1]);
    sc.symbols.push_back(jsym("tile_k", d[2], 1));
    ub("tile_k", d[2]);
    sc.temp_iter.push_back(jop("Div", jc(d[2]), js("tile_k")));
  } else if (f == "attention") {
    if (!need(4)) return LOOM_HIP_EINVAL;
    if (d[3] % 8 || d[3] > 256) {
      err = "constraint_scope: attention is built for head_dim a multiple of 8 up to 256";
      return LOOM_HIP_EUNSUP;
    }
    // the kernel's (padded) head dim and its stages of 64-key K and V blocks
    const long long dk = d[3] <= 64 ? 64 : d[3] <= 128 ? 128 : 256;
    const long long nst = dk > 128 ? 2 : 3;
    sc.symbols.push_back(jsym("tile_b", d[0], 1));
    sc.symbols.push_back(jsym("tile_m", d[1], kTileAlign));
    sc.symbols.push_back(jsym("tile_n", d[2], 1));
    ub("tile_b", d[0]);
    tiled("tile_m", d[1]);
    ub("tile_n", d[2]);
    sc.footprint.push_back(jc(nst * 64 * dk * 2));
    sc.footprint.push_back(jc(nst * 64 * dk * 2));
    sc.hard.push_back(jop("Le", jop("Add", sc.footprint[0], sc.footprint[1]), jc(kLdsBytes)));
    sc.temp_iter.push_back(jop("Div", jc(d[0]), js("tile_b")));
    sc.temp_iter.push_back(jop("Div", jc(d[1]), js("tile_m")));
    sc.seq_iter = jop("Div", jc(d[2]), js("tile_n"));
  } else if (f == "flash_decode") {
    if (!need(4)) return LOOM_HIP_EINVAL;
    if (d[2] % 8 || d[2] > 256) {
      err = "constraint_scope: flash_decode is built for head_dim a multiple of 8 up to 256";
      return LOOM_HIP_EUNSUP;
    }
    sc.symbols.push_back(jsym("tile_b", d[0], 1));
    sc.symbols.push_back(jsym("tile_s", d[3], 1));
    sc.symbols.push_back(jsym("tile_n", d[3], 1));
    sc.hard.push_back(jrange("tile_b", 1, d[0]));
    sc.hard.push_back(jrange("tile_s", 1, d[3]));
    sc.hard.push_back(jrange("tile_n", 1, d[3]));
    sc.temp_iter.push_back(jop("Div", jc(d[0]), js("tile_b")));
    sc.temp_iter.push_back(jop("Div", jc(d[3]), js("tile_s")));
    sc.seq_iter = jop("Div", js("tile_s"), js("tile_n"));
  } else if (f == "helion_mamba2_chunk_scan_kernel") {
    if (!need(7)) return LOOM_HIP_EINVAL;
    if (d[4] > 512 || d[6] > 256 || d[4] % 8 || d[5] % 8 || d[6] % 8 || d[2] % d[3]) {
      err = "constraint_scope: chunk scan is built for chunk_size <= 512, dstate <= 256, "
            "multiples of 8, and nheads a multiple of ngroups";
      return LOOM_HIP_EUNSUP;
    }
    // tile_k is bounded by the example's loom.sym upper_bound (8192,
    // EX(mamba_chunk_scan,00):3), or by the chunk where that is longer: the
    // kernel walks a chunk's keys in 32-key blocks whatever tile_k is
    const long long k_ub = std::max<long long>(8192, d[4]);
    sc.symbols.push_back(jsym("tile_m", d[4], kTileAlign));
    sc.symbols.push_back(jsym("tile_n", d[5], kTileAlign));
    sc.symbols.push_back(jsym("tile_k", k_ub, 1));
    sc.symbols.push_back(jsym("tile_c", d[1], 1));
    sc.symbols.push_back(jsym("tile_b", d[0], 1));
    sc.symbols.push_back(jsym("tile_h", d[2], 1));
    ub("tile_b", d[0]);
    ub("tile_h", d[2]);
    ub("tile_c", d[1]);
    sc.hard.push_back(jop("Eq", js("tile_b"), jc(1)));
    sc.hard.push_back(jop("Eq", js("tile_h"), jc(1)));
    sc.hard.push_back(jop("Eq", js("tile_c"), jc(1)));
    tiled("tile_m", d[4]);
    tiled("tile_n", d[5]);
    ub("tile_k", k_ub);
    sc.temp_iter.push_back(jop("Div", jc(d[4]), js("tile_m")));
    sc.temp_iter.push_back(jop("Div", jc(d[5]), js("tile_n")));
    sc.seq_iter = jop("Div", jc(d[4]), js("tile_k"));
  } else {
    err = "constraint_scope: no gfx950 kernel for function '" + f + "'";
    return LOOM_HIP_EUNSUP;
  }
  return LOOM_HIP_OK;
}

int tensors_of(const std::string& f) {
  if (f == "attention" || f == "flash_decode") return 4;
  if (f == "helion_mamba2_chunk_scan_kernel") return 8;
  return 3;
}

long long ceil_div(long long a, long long b) { return (a + b - 1) / b; }

int copy_out(const std::string& js_, char* out, size_t outlen, char* err, size_t errlen,
             const char* fn) {
  if (!out || outlen <= js_.size())
    return fail(err, errlen, LOOM_HIP_EINVAL, "%s: output buffer needs %zu bytes", fn,
                js_.size() + 1);
  memcpy(out, js_.c_str(), js_.size() + 1);
  if (err && errlen) err[0] = '\0';
  return LOOM_HIP_OK;
}

thread_local bool g_validate_only = false;

template <bool F16>
int dispatch_impl(const char* variant, void* const* tensors, int ntensors,
                      const int64_t* dims, int ndims, float scale, int causal,
                      void* workspace, size_t workspace_bytes, void* stream, char* err,
                      size_t errlen) {
  if (!variant || (ntensors > 0 && !tensors) || (ndims > 0 && !dims))
    return fail(err, errlen, LOOM_HIP_EINVAL, "dispatch: null argument");
  std::string f, perr;
  int64_t t[LOOM_HIP_NTILES];
  int rc = parse_variant(variant, f, t, perr);
  if (rc) return fail(err, errlen, rc, "dispatch: %s", perr.c_str());
  if (!known_function(f))
    return fail(err, errlen, LOOM_HIP_EUNSUP, "dispatch: no gfx950 kernel for function '%s'",
                f.c_str());
  auto shape = [&](int nt, int nd) {
    if (ntensors != nt || ndims != nd)
      return fail(err, errlen, LOOM_HIP_EINVAL,
                  "dispatch: %s takes %d tensors and %d extents (got %d and %d)", f.c_str(), nt,
                  nd, ntensors, ndims);
    return (int)LOOM_HIP_OK;
  };
  if (f == "matmul") {
    if ((rc = shape(3, 3)) || (rc = need_tiles(f, t, {1, 2, 3}, err, errlen))) return rc;
    const auto fn = F16 ? loom_hip_matmul_f16 : loom_hip_matmul;
    return fn(tensors[0], tensors[1], tensors[2], dims[0], dims[1], dims[2], t[LOOM_HIP_TILE_M],
              t[LOOM_HIP_TILE_N], t[LOOM_HIP_TILE_K], stream, err, errlen);
  }
  if (f == "batch_matmul") {
    if ((rc = shape(3, 4)) || (rc = need_tiles(f, t, {0, 1, 2, 3}, err, errlen))) return rc;
    const auto fn = F16 ? loom_hip_batch_matmul_f16 : loom_hip_batch_matmul;
    return fn(tensors[0], tensors[1], tensors[2], dims[0], dims[1], dims[2], dims[3],
              t[LOOM_HIP_TILE_B], t[LOOM_HIP_TILE_M], t[LOOM_HIP_TILE_N], t[LOOM_HIP_TILE_K],
              stream, err, errlen);
  }
  if (f == "split_k_matmul_gather") {
    if ((rc = shape(3, 3)) || (rc = need_tiles(f, t, {1, 2, 3}, err, errlen))) return rc;
    const auto fn = F16 ? loom_hip_split_k_matmul_gather_f16 : loom_hip_split_k_matmul_gather;
    return fn(tensors[0], tensors[1], tensors[2], workspace, workspace_bytes, dims[0], dims[1],
              dims[2], t[LOOM_HIP_TILE_M], t[LOOM_HIP_TILE_N], t[LOOM_HIP_TILE_K], stream, err,
              errlen);
  }
  if (f == "attention") {
    if ((rc = shape(4, 4)) || (rc = need_tiles(f, t, {0, 1, 2}, err, errlen))) return rc;
    const auto fn = F16 ? loom_hip_attention_f16 : loom_hip_attention;
    return fn(tensors[0], tensors[1], tensors[2], tensors[3], dims[0], dims[1], dims[2], dims[3],
              scale, causal, t[LOOM_HIP_TILE_B], t[LOOM_HIP_TILE_M], t[LOOM_HIP_TILE_N], stream,
              err, errlen);
  }
  if (f == "flash_decode") {
    if ((rc = shape(4, 4)) || (rc = need_tiles(f, t, {0, 2, 4}, err, errlen))) return rc;
    const auto fn = F16 ? loom_hip_flash_decode_f16 : loom_hip_flash_decode;
    return fn(tensors[0], tensors[1], tensors[2], tensors[3], workspace, workspace_bytes, dims[0],
              dims[1], dims[2], dims[3], scale, t[LOOM_HIP_TILE_B], t[LOOM_HIP_TILE_S],
              t[LOOM_HIP_TILE_N], stream, err, errlen);
  }
  // helion_mamba2_chunk_scan_kernel
  if ((rc = shape(8, 7)) || (rc = need_tiles(f, t, {0, 1, 2, 3, 5, 6}, err, errlen))) return rc;
  const auto fn =
      F16 ? loom_hip_helion_mamba2_chunk_scan_kernel_f16 : loom_hip_helion_mamba2_chunk_scan_kernel;
  return fn(tensors[0], tensors[1], tensors[2], tensors[3], tensors[4], tensors[5], tensors[6],
            tensors[7], dims[0], dims[1], dims[2], dims[3], dims[4], dims[5], dims[6],
            t[LOOM_HIP_TILE_B], t[LOOM_HIP_TILE_H], t[LOOM_HIP_TILE_C], t[LOOM_HIP_TILE_M],
            t[LOOM_HIP_TILE_N], t[LOOM_HIP_TILE_K], stream, err, errlen);
}


}  // namespace

// entry points check this before launching (declared in csrc/common.h)
bool& loom_validate_only_flag() { return g_validate_only; }

extern "C" {

const char* loom_hip_version(void) { return LOOM_HIP_VERSION_STRING; }

int loom_hip_check_variant(const char* variant, const int64_t* dims, int ndims, char* err,
                           size_t errlen) {
  if (!variant) return fail(err, errlen, LOOM_HIP_EINVAL, "check_variant: null variant");
  std::string f, perr;
  int64_t t[LOOM_HIP_NTILES];
  int rc = parse_variant(variant, f, t, perr);
  if (rc) return fail(err, errlen, rc, "check_variant: %s", perr.c_str());
  // stand-in pointers: aligned, never dereferenced (nothing launches)
  void* fake[8];
  for (auto& x : fake) x = reinterpret_cast<void*>(uintptr_t(1) << 20);
  struct Guard {
    Guard() { g_validate_only = true; }
    ~Guard() { g_validate_only = false; }
  } guard;
  return loom_hip_dispatch(variant, fake, tensors_of(f), dims, ndims, 1.0f, 0, fake[0],
                           ~(size_t)0, nullptr, err, errlen);
}

int loom_hip_constraint_scope(const char* func, const int64_t* dims, int ndims, char* out,
                              size_t outlen, char* err, size_t errlen) {
  if (!func || (ndims > 0 && !dims))
    return fail(err, errlen, LOOM_HIP_EINVAL, "constraint_scope: null argument");
  const std::string f = std::string(func).substr(0, std::string(func).find("__"));
  Scope sc;
  std::string perr;
  const int rc = build_scope(f, dims, ndims, sc, perr);
  if (rc) return fail(err, errlen, rc, "%s", perr.c_str());
  std::string j = std::string("{\"variant_name\":\"") + func + "\",\"constraint_scope\":{" +
                  "\"metadata\":{\"datatype\":\"bf16\",\"target\":\"gfx950\",\"memory\":\"LDS\"," +
                  "\"capacity_bytes\":" + std::to_string(kLdsBytes) + ",\"booleans\":[]," +
                  "\"iter_num\":{\"temp_iter\":[";
  for (size_t i = 0; i < sc.temp_iter.size(); ++i) j += (i ? "," : "") + sc.temp_iter[i];
  j += "]";
  if (!sc.seq_iter.empty()) j += ",\"seq_iter\":" + sc.seq_iter;
  j += "},\"L1_footprint\":[";
  for (size_t i = 0; i < sc.footprint.size(); ++i) j += (i ? "," : "") + sc.footprint[i];
  j += "],\"symbols\":{";
  for (size_t i = 0; i < sc.symbols.size(); ++i) j += (i ? "," : "") + sc.symbols[i];
  j += "}},\"hard_constraints\":[";
  for (size_t i = 0; i < sc.hard.size(); ++i) j += (i ? "," : "") + sc.hard[i];
  j += "]}}";
  return copy_out(j, out, outlen, err, errlen, "constraint_scope");
}

int loom_hip_preferred_block_sizes(const char* func, const int64_t* dims, int ndims, char* out,
                                   size_t outlen, char* err, size_t errlen) {
  if (!func || (ndims > 0 && !dims))
    return fail(err, errlen, LOOM_HIP_EINVAL, "preferred_block_sizes: null argument");
  const std::string f = std::string(func).substr(0, std::string(func).find("__"));
  Scope sc;
  std::string perr;
  int rc = build_scope(f, dims, ndims, sc, perr);   // validates f and the extents
  if (rc) return fail(err, errlen, rc, "%s", perr.c_str());
  const int64_t* d = dims;
  constexpr long long kCUs = 256;
  std::map<std::string, long long> b;
  // a workgroup tile T bound within natural_ub: T itself, or the whole
  // extent when that is below T (it runs as T)
  auto bound = [](long long T, long long extent) { return std::min(T, extent); };
  // largest square GEMM tile that still gives every CU a workgroup, among
  // those a binding can name for these extents
  auto gemm_pick = [&](long long M, long long N, long long z) {
    auto nameable = [&](long long T, long long E) {
      return T <= E || (T == 64 && E < 64) || (T == 128 && E > 64 && E < 128) ||
             (T == 256 && E > 128 && E < 256);
    };
    for (long long t : {256LL, 128LL})
      if (nameable(t, M) && nameable(t, N) && ceil_div(M, t) * ceil_div(N, t) * z >= kCUs) {
        b["tile_m"] = bound(t, M);
        b["tile_n"] = bound(t, N);
        return;
      }
    // 64 is nameable on every axis (64 itself, or an extent below it)
    b["tile_m"] = bound(64, M);
    b["tile_n"] = bound(64, N);
  };
  if (f == "matmul") {
    gemm_pick(d[0], d[1], 1);
    b["tile_k"] = std::min<long long>(64, d[2]);
  } else if (f == "batch_matmul") {
    b["tile_b"] = 1;
    gemm_pick(d[1], d[2], d[0]);
    b["tile_k"] = std::min<long long>(64, d[3]);
  } else if (f == "split_k_matmul_gather") {
    // 128x128 tiles (64x64 when M or N is small), enough K slabs to cover
    // the CUs, slabs a whole number of the pipelined kernel's rounds (256
    // deep for 128 tiles, 512 for 64) when K allows
    const long long t = (d[0] >= 128 && d[1] >= 128) ? 128 : 64;
    const long long round = t == 128 ? 256 : 512;
    b["tile_m"] = bound(t, d[0]);
    b["tile_n"] = bound(t, d[1]);
    const long long tiles = ceil_div(d[0], t) * ceil_div(d[1], t);
    const long long step = d[2] >= round ? round : 64;
    const long long S = std::max(1LL, std::min(ceil_div(kCUs, tiles), ceil_div(d[2], step)));
    b["tile_k"] = std::min<long long>(d[2], ceil_div(ceil_div(d[2], S), step) * step);
  } else if (f == "attention") {
    b["tile_b"] = 1;
    // 256 query rows (128 for head dims above 128), or the largest built
    // tile within a shorter Sq (Sq itself below 64)
    const long long top = d[3] > 128 ? 128 : 256;
    b["tile_m"] = d[1] >= top ? top : d[1] >= 192 ? 192 : d[1] >= 128 ? 128 : d[1] >= 64 ? 64 : d[1];
    b["tile_n"] = std::min<long long>(64, d[2]);
  } else if (f == "flash_decode") {
    b["tile_b"] = 1;
    // one workgroup per (batch, split): about one per CU
    const long long ns = std::max(1LL, ceil_div(kCUs, d[0]));
    b["tile_s"] = std::min<long long>(d[3], ceil_div(ceil_div(d[3], ns), 64) * 64);
    b["tile_n"] = std::min<long long>(128, b["tile_s"]);
  } else {  // helion_mamba2_chunk_scan_kernel
    b["tile_b"] = b["tile_h"] = b["tile_c"] = 1;
    // one m tile per chunk: the chunk itself (it runs as the covering tile)
    b["tile_m"] = d[4];
    b["tile_n"] = d[5] >= 64 ? 64 : d[5] >= 32 ? 32 : d[5] >= 16 ? 16 : d[5];
    b["tile_k"] = std::min<long long>(64, d[4]);
  }
  std::string j = "{";
  bool first = true;
  for (const auto& kv : b) {
    j += (first ? "\"" : ",\"") + kv.first + "\":" + std::to_string(kv.second);
    first = false;
  }
  j += "}";
  return copy_out(j, out, outlen, err, errlen, "preferred_block_sizes");
}

int loom_hip_materialize_variants(const char* block_sizes_json, const char* const* funcs,
                                  int nfuncs, char* out, size_t outlen, char* err,
                                  size_t errlen) {
  if (!block_sizes_json || (nfuncs > 0 && !funcs) || nfuncs < 0)
    return fail(err, errlen, LOOM_HIP_EINVAL, "materialize_variants: null argument");
  for (int i = 0; i < nfuncs; ++i)
    if (!funcs[i]) return fail(err, errlen, LOOM_HIP_EINVAL, "materialize_variants: null name");
  BlockSizes bs;
  std::string perr;
  if (!parse_block_sizes(block_sizes_json, bs, perr))
    return fail(err, errlen, LOOM_HIP_EINVAL, "%s", perr.c_str());
  const bool external = block_sizes_json[0] != '\0';

  std::vector<std::string> order(funcs, funcs + nfuncs);
  if (external) {
    // "ALL": every listed function without its own binding, in list order;
    // it replaces the candidate order by exactly those functions
    if (bs.has_all) {
      bs.candidate_order.clear();
      for (const auto& f : order) {
        bool have = false;
        for (const auto& e : bs.funcs) have |= e.first == f;
        if (!have) {
          bs.funcs.emplace_back(f, bs.all);
          bs.candidate_order.push_back(f);
        }
      }
    }
    // stable sort by candidate rank; unranked functions keep list order last
    std::map<std::string, size_t> rank;
    for (size_t r = 0; r < bs.candidate_order.size(); ++r) rank[bs.candidate_order[r]] = r;
    auto rank_of = [&](const std::string& f) {
      auto it = rank.find(f);
      return it == rank.end() ? rank.size() : it->second;
    };
    std::stable_sort(order.begin(), order.end(), [&](const std::string& a, const std::string& b) {
      return rank_of(a) < rank_of(b);
    });
  }

  std::string names;
  for (const auto& f : order) {
    std::vector<Binding> bl;
    if (external) {
      for (const auto& e : bs.funcs)
        if (e.first == f) bl = e.second;
    } else {
      // mapping variants ("matmul__x8_y1y8__...") carry their base's symbols
      const std::vector<std::string>* syms = known_symbols(f.substr(0, f.find("__")));
      if (!syms || syms->empty()) continue;  // symbols unknown: nothing to bind
      bl.push_back(placeholder_binding(*syms));
    }
    std::set<std::string> used;  // names are unique per function's module
    for (size_t bi = 0; bi < bl.size(); ++bi) {
      std::string n = f + suffix_of(bl[bi]);
      if (used.count(n)) {
        const std::string base = n;
        unsigned combo = (unsigned)bi;
        do {
          ++combo;
          n = base + "__combo" + std::to_string(combo);
        } while (used.count(n));
      }
      used.insert(n);
      names += n;
      names += '\n';
    }
  }
  if (!out || outlen <= names.size())
    return fail(err, errlen, LOOM_HIP_EINVAL,
                "materialize_variants: output buffer needs %zu bytes", names.size() + 1);
  memcpy(out, names.c_str(), names.size() + 1);
  if (err && errlen) err[0] = '\0';
  return LOOM_HIP_OK;
}

int loom_hip_parse_variant(const char* variant, char* func, size_t funclen, int64_t* tiles,
                           char* err, size_t errlen) {
  if (!variant || !tiles)
    return fail(err, errlen, LOOM_HIP_EINVAL, "parse_variant: null argument");
  std::string f, perr;
  const int rc = parse_variant(variant, f, tiles, perr);
  if (rc) return fail(err, errlen, rc, "%s", perr.c_str());
  if (func) {
    if (funclen <= f.size())
      return fail(err, errlen, LOOM_HIP_EINVAL, "parse_variant: function buffer too small");
    memcpy(func, f.c_str(), f.size() + 1);
  }
  if (err && errlen) err[0] = '\0';
  return LOOM_HIP_OK;
}

int loom_hip_workspace_bytes(const char* variant, const int64_t* dims, int ndims,
                             size_t* bytes, char* err, size_t errlen) {
  if (!variant || !bytes || (ndims > 0 && !dims))
    return fail(err, errlen, LOOM_HIP_EINVAL, "workspace_bytes: null argument");
  std::string f, perr;
  int64_t t[LOOM_HIP_NTILES];
  int rc = parse_variant(variant, f, t, perr);
  if (rc) return fail(err, errlen, rc, "workspace_bytes: %s", perr.c_str());
  if (!known_function(f))
    return fail(err, errlen, LOOM_HIP_EUNSUP,
                "workspace_bytes: no gfx950 kernel for function '%s'", f.c_str());
  const int nd = f == "split_k_matmul_gather" || f == "matmul" ? 3
                 : f == "helion_mamba2_chunk_scan_kernel" ? 7 : 4;
  if (ndims != nd)
    return fail(err, errlen, LOOM_HIP_EINVAL, "workspace_bytes: %s takes %d extents (got %d)",
                f.c_str(), nd, ndims);
  for (int i = 0; i < nd; ++i)
    if (dims[i] <= 0)
      return fail(err, errlen, LOOM_HIP_EINVAL, "workspace_bytes: extents must be positive");
  size_t n = 0;
  if (f == "split_k_matmul_gather") {
    if ((rc = need_tiles(f, t, {3}, err, errlen))) return rc;
    n = loom_hip_split_k_workspace_bytes(dims[0], dims[1], dims[2], t[LOOM_HIP_TILE_K]);
  } else if (f == "flash_decode") {
    if ((rc = need_tiles(f, t, {4}, err, errlen))) return rc;
    n = loom_hip_flash_decode_workspace_bytes(dims[0], dims[1], dims[2], dims[3],
                                              t[LOOM_HIP_TILE_S]);
  }
  if (n == SIZE_MAX)
    return fail(err, errlen, LOOM_HIP_EINVAL, "workspace_bytes: %s workspace too large",
                f.c_str());
  *bytes = n;
  if (err && errlen) err[0] = '\0';
  return LOOM_HIP_OK;
}

int loom_hip_dispatch(const char* variant, void* const* tensors, int ntensors,
                      const int64_t* dims, int ndims, float scale, int causal,
                      void* workspace, size_t workspace_bytes, void* stream, char* err,
                      size_t errlen) {
  return dispatch_impl<false>(variant, tensors, ntensors, dims, ndims, scale, causal, workspace,
                              workspace_bytes, stream, err, errlen);
}

int loom_hip_dispatch_f16(const char* variant, void* const* tensors, int ntensors,
                          const int64_t* dims, int ndims, float scale, int causal,
                          void* workspace, size_t workspace_bytes, void* stream, char* err,
                          size_t errlen) {
  return dispatch_impl<true>(variant, tensors, ntensors, dims, ndims, scale, causal, workspace,
                             workspace_bytes, stream, err, errlen);
}

int loom_hip_hw_spec(int device, char* out, size_t outlen, char* err, size_t errlen) {
  // The machine model the gfx950 constraint scopes are written against
  // (loom_hip_constraint_scope): the LDS capacity of their footprint
  // constraint, the workgroup tiles the kernels build, the MFMA shapes the
  // tiles are multiples of; with device >= 0, also what that device reports.
  std::string j = "{\"target\":\"gfx950\",\"wave_size\":64,\"simds_per_cu\":4,"
                  "\"vgprs_per_simd_lane\":512,\"max_workgroup_threads\":1024,"
                  "\"lds_bytes_per_workgroup\":" + std::to_string(kLdsBytes) + ","
                  "\"tile_alignment\":" + std::to_string(kTileAlign) + ","
                  "\"xcds\":8,\"mfma\":[{\"op\":\"v_mfma_f32_16x16x32_bf16\",\"m\":16,\"n\":16,"
                  "\"k\":32,\"cycles\":16},{\"op\":\"v_mfma_f32_16x16x32_f16\",\"m\":16,\"n\":16,"
                  "\"k\":32,\"cycles\":16}],"
                  "\"published\":{\"compute_units\":256,\"clock_mhz\":2400,"
                  "\"bf16_dense_tflops\":2516.6,\"hbm_gbs\":8000,\"hbm_bytes\":309237645312,"
                  "\"infinity_cache_bytes\":268435456},"
                  "\"built_tiles\":{\"matmul\":{\"tile_m\":[64,128,256],\"tile_n\":[64,128,256]},"
                  "\"batch_matmul\":{\"tile_m\":[64,128,256],\"tile_n\":[64,128,256]},"
                  "\"split_k_matmul_gather\":{\"tile_m\":[64,128,256],\"tile_n\":[64,128,256]},"
                  "\"attention\":{\"tile_m\":[64,128,192,256]},"
                  "\"helion_mamba2_chunk_scan_kernel\":{\"tile_m\":[64,128,192,256],"
                  "\"tile_n\":[16,32,64]}}";
  if (device >= 0) {
    hipDeviceProp_t pr;
    const hipError_t e = hipGetDeviceProperties(&pr, device);
    if (e != hipSuccess)
      return fail(err, errlen, LOOM_HIP_EHIP, "hw_spec: device %d: %s", device,
                  hipGetErrorString(e));
    std::string arch(pr.gcnArchName), name(pr.name);
    for (auto* t : {&arch, &name})
      for (char& ch : *t)
        if (ch == '"' || ch == '\\' || (unsigned char)ch < 0x20) ch = ' ';
    j += ",\"device\":{\"index\":" + std::to_string(device) + ",\"name\":\"" + name +
         "\",\"arch\":\"" + arch + "\",\"compute_units\":" +
         std::to_string(pr.multiProcessorCount) + ",\"lds_bytes_per_cu\":" +
         std::to_string(pr.maxSharedMemoryPerMultiProcessor) + ",\"lds_bytes_per_workgroup\":" +
         std::to_string(pr.sharedMemPerBlock) + ",\"l2_bytes\":" + std::to_string(pr.l2CacheSize) +
         ",\"global_bytes\":" + std::to_string(pr.totalGlobalMem) + ",\"clock_mhz\":" +
         std::to_string(pr.clockRate / 1000) + ",\"warp_size\":" + std::to_string(pr.warpSize) +
         "}";
  }
  j += "}";
  return copy_out(j, out, outlen, err, errlen, "hw_spec");
}

}  // extern "C"
