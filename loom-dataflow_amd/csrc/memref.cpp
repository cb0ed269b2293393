// memref.cpp -- the C ABI over MLIR ranked-memref descriptors.
//
// A materialized variant is an MLIR function over memrefs
// (examples/mm/IR/00_from_helion_frontend.mlir:2, ...); a caller lowered
// through MLIR's C interface holds each argument as a ranked descriptor
// {allocated, aligned, offset, sizes[R], strides[R]} and passes a pointer to
// it (the `_mlir_ciface_` convention of MLIR's C runner utilities).  The
// entry points here take exactly those structs (loom_memref<R>_t in
// include/loom_hip.h), read the extents from their sizes, honour the element
// offset, and launch through the pointer entry points.  Layouts the kernels
// do not address -- any stride other than the row-major contiguous one, the
// innermost included -- are refused with LOOM_HIP_EINVAL and a message that
// names the argument; so are shapes that disagree between arguments.
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/loom_hip.h"

bool& loom_validate_only_flag();   // abi.cpp: entry points validate, launch nothing

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

// One memref argument seen through its descriptor, whatever its rank: the
// descriptor layout is {allocated, aligned, offset, sizes[R], strides[R]}.
struct View {
  const void* aligned;
  int64_t offset;
  const int64_t* sizes;
  const int64_t* strides;
};

View view_of(const void* desc, int rank) {
  const char* p = static_cast<const char*>(desc);
  View v;
  std::memcpy(&v.aligned, p + sizeof(void*), sizeof(void*));
  std::memcpy(&v.offset, p + 2 * sizeof(void*), sizeof(int64_t));
  v.sizes = reinterpret_cast<const int64_t*>(p + 2 * sizeof(void*) + sizeof(int64_t));
  v.strides = v.sizes + rank;
  return v;
}

// Argument kinds: the call's 16-bit element type, or a side tensor (fp32 in
// the bf16 variants, f16 in the f16 variants: mamba's dt, dA_cumsum, D,
// prev_states_T).
enum Kind { kElem, kSide };

struct Arg {
  const char* name;
  int rank;
  Kind kind;
};

struct Func {
  const char* name;
  std::vector<Arg> args;
};

const std::vector<Func>& funcs() {
  static const std::vector<Func> f = {
      {"matmul", {{"x", 2, kElem}, {"y", 2, kElem}, {"out", 2, kElem}}},
      {"batch_matmul", {{"arg0", 3, kElem}, {"arg1", 3, kElem}, {"arg2", 3, kElem}}},
      {"split_k_matmul_gather", {{"a", 2, kElem}, {"b", 2, kElem}, {"out", 2, kElem}}},
      {"attention", {{"k", 3, kElem}, {"v", 3, kElem}, {"q", 3, kElem}, {"out", 3, kElem}}},
      {"flash_decode", {{"k", 3, kElem}, {"v", 3, kElem}, {"q", 3, kElem}, {"out", 3, kElem}}},
      {"helion_mamba2_chunk_scan_kernel",
       {{"cb", 5, kElem},
        {"x", 4, kElem},
        {"dt", 4, kSide},
        {"dA_cumsum", 4, kSide},
        {"C", 4, kElem},
        {"D", 1, kSide},
        {"prev_states_T", 5, kSide},
        {"out", 4, kElem}}},
  };
  return f;
}

const Func* find(const std::string& name) {
  for (const auto& f : funcs())
    if (name == f.name) return &f;
  return nullptr;
}

// The extents of a call in loom_hip_dispatch's order, read from the input
// descriptors, and the shape every argument must then have.
std::vector<int64_t> dims_of(const std::string& f, const std::vector<View>& v) {
  if (f == "matmul" || f == "split_k_matmul_gather")
    return {v[0].sizes[0], v[1].sizes[1], v[0].sizes[1]};                    // M, N, K
  if (f == "batch_matmul")
    return {v[0].sizes[0], v[0].sizes[1], v[1].sizes[2], v[0].sizes[2]};     // B, M, N, K
  if (f == "attention")
    return {v[0].sizes[0], v[2].sizes[1], v[0].sizes[2], v[0].sizes[1]};     // BH, Sq, Skv, D
  if (f == "flash_decode")
    return {v[0].sizes[0], v[2].sizes[1], v[0].sizes[1], v[0].sizes[2]};     // B, H, D, S
  // chunk scan: b, nc, H, G, Q, P, N
  return {v[0].sizes[0], v[0].sizes[1], v[1].sizes[1], v[0].sizes[2],
          v[0].sizes[3], v[1].sizes[3], v[4].sizes[3]};
}

std::vector<std::vector<int64_t>> shapes_of(const std::string& f, const std::vector<int64_t>& d) {
  if (f == "matmul" || f == "split_k_matmul_gather")
    return {{d[0], d[2]}, {d[2], d[1]}, {d[0], d[1]}};
  if (f == "batch_matmul")
    return {{d[0], d[1], d[3]}, {d[0], d[3], d[2]}, {d[0], d[1], d[2]}};
  if (f == "attention")
    return {{d[0], d[3], d[2]}, {d[0], d[2], d[3]}, {d[0], d[1], d[3]}, {d[0], d[1], d[3]}};
  if (f == "flash_decode")
    return {{d[0], d[2], d[3]}, {d[0], d[3], d[2]}, {d[0], d[1], d[2]}, {d[0], d[1], d[2]}};
  const int64_t b = d[0], nc = d[1], H = d[2], G = d[3], Q = d[4], P = d[5], N = d[6];
  return {{b, nc, G, Q, Q}, {b, H, nc * Q, P}, {b, H, nc, Q},    {b, H, nc, Q},
          {b, G, nc * Q, N}, {H},               {b, nc, H, N, P}, {b, H, nc * Q, P}};
}

std::string list(const int64_t* a, int n) {
  std::string s = "[";
  for (int i = 0; i < n; ++i) s += (i ? ", " : "") + std::to_string((long long)a[i]);
  return s + "]";
}

// Unpacks and checks every descriptor of `f`: ranks come from the function's
// signature, extents from the inputs; each argument must match its expected
// shape, sit at a non-negative offset from a non-null aligned pointer and be
// row-major contiguous (innermost stride 1, each outer stride the product of
// the sizes inside it; dimensions of size 1 are never stepped over, so their
// strides are not constrained).  On success `ptrs` holds the element-offset
// data pointers and `dims` the extents.
int unpack(const Func& f, const void* const* descs, int ndescs, bool f16,
           std::vector<const void*>& ptrs, std::vector<int64_t>& dims, char* err, size_t errlen) {
  const int n = (int)f.args.size();
  if (!descs || ndescs != n)
    return fail(err, errlen, LOOM_HIP_EINVAL, "%s: takes %d memref descriptors, got %d", f.name, n,
                ndescs);
  std::vector<View> v(n);
  for (int i = 0; i < n; ++i) {
    if (!descs[i])
      return fail(err, errlen, LOOM_HIP_EINVAL, "%s: %s: null descriptor", f.name, f.args[i].name);
    v[i] = view_of(descs[i], f.args[i].rank);
    // bounded before any arithmetic on them (no extent reaches 2^31)
    for (int r = 0; r < f.args[i].rank; ++r)
      if (v[i].sizes[r] < 0 || v[i].sizes[r] >= ((int64_t)1 << 31))
        return fail(err, errlen, LOOM_HIP_EINVAL, "%s: %s: size %lld out of range", f.name,
                    f.args[i].name, (long long)v[i].sizes[r]);
    if (v[i].offset < 0 || v[i].offset >= ((int64_t)1 << 56))
      return fail(err, errlen, LOOM_HIP_EINVAL, "%s: %s: %s offset %lld", f.name, f.args[i].name,
                  v[i].offset < 0 ? "negative" : "out-of-range", (long long)v[i].offset);
  }
  dims = dims_of(f.name, v);
  const auto shapes = shapes_of(f.name, dims);
  ptrs.assign(n, nullptr);
  for (int i = 0; i < n; ++i) {
    const Arg& a = f.args[i];
    const View& m = v[i];
    const std::vector<int64_t>& want = shapes[i];
    for (int r = 0; r < a.rank; ++r)
      if (m.sizes[r] != want[r])
        return fail(err, errlen, LOOM_HIP_EINVAL,
                    "%s: %s: sizes %s do not match the call (expected %s)", f.name, a.name,
                    list(m.sizes, a.rank).c_str(), list(want.data(), a.rank).c_str());
    if (!m.aligned)
      return fail(err, errlen, LOOM_HIP_EINVAL, "%s: %s: null aligned pointer", f.name, a.name);
    int64_t expect = 1;
    for (int r = a.rank - 1; r >= 0; --r) {
      if (m.sizes[r] != 1 && m.strides[r] != expect) {
        std::vector<int64_t> rowmajor(a.rank);
        int64_t e = 1;
        for (int q = a.rank - 1; q >= 0; --q) {
          rowmajor[q] = e;
          if (__builtin_mul_overflow(e, m.sizes[q], &e)) e = INT64_MAX;
        }
        return fail(err, errlen, LOOM_HIP_EINVAL,
                    "%s: %s: strides %s are not the row-major contiguous layout %s the kernels "
                    "address%s",
                    f.name, a.name, list(m.strides, a.rank).c_str(),
                    list(rowmajor.data(), a.rank).c_str(),
                    r == a.rank - 1 ? " (innermost stride must be 1)" : "");
      }
      if (__builtin_mul_overflow(expect, m.sizes[r], &expect))
        return fail(err, errlen, LOOM_HIP_EINVAL, "%s: %s: too many elements", f.name, a.name);
    }
    const size_t esize = (a.kind == kSide && !f16) ? 4 : 2;
    ptrs[i] = static_cast<const char*>(m.aligned) + m.offset * (int64_t)esize;
  }
  return LOOM_HIP_OK;
}

// The pointer entry point of `f` with the unpacked arguments and its tiles.
// `t` holds tiles in the LOOM_HIP_TILE_* slots.
int launch(const Func& f, bool f16, const std::vector<const void*>& p, const std::vector<int64_t>& d,
           const int64_t* t, float scale, int causal, void* workspace, size_t workspace_bytes,
           void* stream, char* err, size_t errlen) {
  std::vector<void*> tensors(p.size());
  for (size_t i = 0; i < p.size(); ++i) tensors[i] = const_cast<void*>(p[i]);
  const std::string n = f.name;
  const int64_t tb = t[LOOM_HIP_TILE_B], tm = t[LOOM_HIP_TILE_M], tn = t[LOOM_HIP_TILE_N],
                tk = t[LOOM_HIP_TILE_K], ts = t[LOOM_HIP_TILE_S], th = t[LOOM_HIP_TILE_H],
                tc = t[LOOM_HIP_TILE_C];
  void** a = tensors.data();
  if (n == "matmul")
    return (f16 ? loom_hip_matmul_f16 : loom_hip_matmul)(a[0], a[1], a[2], d[0], d[1], d[2], tm,
                                                         tn, tk, stream, err, errlen);
  if (n == "batch_matmul")
    return (f16 ? loom_hip_batch_matmul_f16 : loom_hip_batch_matmul)(
        a[0], a[1], a[2], d[0], d[1], d[2], d[3], tb, tm, tn, tk, stream, err, errlen);
  if (n == "split_k_matmul_gather")
    return (f16 ? loom_hip_split_k_matmul_gather_f16 : loom_hip_split_k_matmul_gather)(
        a[0], a[1], a[2], workspace, workspace_bytes, d[0], d[1], d[2], tm, tn, tk, stream, err,
        errlen);
  if (n == "attention")
    return (f16 ? loom_hip_attention_f16 : loom_hip_attention)(
        a[0], a[1], a[2], a[3], d[0], d[1], d[2], d[3], scale, causal, tb, tm, tn, stream, err,
        errlen);
  if (n == "flash_decode")
    return (f16 ? loom_hip_flash_decode_f16 : loom_hip_flash_decode)(
        a[0], a[1], a[2], a[3], workspace, workspace_bytes, d[0], d[1], d[2], d[3], scale, tb, ts,
        tn, stream, err, errlen);
  return (f16 ? loom_hip_helion_mamba2_chunk_scan_kernel_f16
              : loom_hip_helion_mamba2_chunk_scan_kernel)(
      a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7], d[0], d[1], d[2], d[3], d[4], d[5], d[6], tb,
      th, tc, tm, tn, tk, stream, err, errlen);
}

int call(const char* fname, bool f16, const void* const* descs, int n, const int64_t* tiles,
         float scale, int causal, void* workspace, size_t workspace_bytes, void* stream, char* err,
         size_t errlen) {
  const Func* f = find(fname);
  std::vector<const void*> p;
  std::vector<int64_t> d;
  int rc = unpack(*f, descs, n, f16, p, d, err, errlen);
  if (rc) return rc;
  return launch(*f, f16, p, d, tiles, scale, causal, workspace, workspace_bytes, stream, err,
                errlen);
}

struct Tiles {
  int64_t t[LOOM_HIP_NTILES];
  Tiles() {
    for (auto& x : t) x = -1;
  }
};

int dispatch_memref(const char* variant, const void* const* descs, int ndescs, bool f16,
                    float scale, int causal, void* workspace, size_t workspace_bytes, void* stream,
                    char* err, size_t errlen) {
  if (!variant) return fail(err, errlen, LOOM_HIP_EINVAL, "dispatch_memref: null variant");
  char fname[256];
  Tiles t;
  int rc = loom_hip_parse_variant(variant, fname, sizeof fname, t.t, err, errlen);
  if (rc) return rc;
  const Func* f = find(fname);
  if (!f)
    return fail(err, errlen, LOOM_HIP_EUNSUP, "dispatch_memref: no gfx950 kernel for function '%s'",
                fname);
  std::vector<const void*> p;
  std::vector<int64_t> d;
  if ((rc = unpack(*f, descs, ndescs, f16, p, d, err, errlen))) return rc;
  // the pointer dispatcher: it checks that the name binds every tile symbol
  // the entry point takes, then launches
  std::vector<void*> tensors(p.size());
  for (size_t i = 0; i < p.size(); ++i) tensors[i] = const_cast<void*>(p[i]);
  return (f16 ? loom_hip_dispatch_f16 : loom_hip_dispatch)(
      variant, tensors.data(), (int)tensors.size(), d.data(), (int)d.size(), scale, causal,
      workspace, workspace_bytes, stream, err, errlen);
}

}  // namespace

extern "C" {

int loom_hip_ciface_matmul(const loom_memref2_t* x, const loom_memref2_t* y,
                           const loom_memref2_t* out, int64_t tile_m, int64_t tile_n,
                           int64_t tile_k, void* stream, char* err, size_t errlen) {
  const void* d[] = {x, y, out};
  Tiles t;
  t.t[LOOM_HIP_TILE_M] = tile_m, t.t[LOOM_HIP_TILE_N] = tile_n, t.t[LOOM_HIP_TILE_K] = tile_k;
  return call("matmul", false, d, 3, t.t, 0.f, 0, nullptr, 0, stream, err, errlen);
}
int loom_hip_ciface_matmul_f16(const loom_memref2_t* x, const loom_memref2_t* y,
                               const loom_memref2_t* out, int64_t tile_m, int64_t tile_n,
                               int64_t tile_k, void* stream, char* err, size_t errlen) {
  const void* d[] = {x, y, out};
  Tiles t;
  t.t[LOOM_HIP_TILE_M] = tile_m, t.t[LOOM_HIP_TILE_N] = tile_n, t.t[LOOM_HIP_TILE_K] = tile_k;
  return call("matmul", true, d, 3, t.t, 0.f, 0, nullptr, 0, stream, err, errlen);
}

int loom_hip_ciface_batch_matmul(const loom_memref3_t* arg0, const loom_memref3_t* arg1,
                                 const loom_memref3_t* arg2, int64_t tile_b, int64_t tile_m,
                                 int64_t tile_n, int64_t tile_k, void* stream, char* err,
                                 size_t errlen) {
  const void* d[] = {arg0, arg1, arg2};
  Tiles t;
  t.t[LOOM_HIP_TILE_B] = tile_b, t.t[LOOM_HIP_TILE_M] = tile_m, t.t[LOOM_HIP_TILE_N] = tile_n;
  t.t[LOOM_HIP_TILE_K] = tile_k;
  return call("batch_matmul", false, d, 3, t.t, 0.f, 0, nullptr, 0, stream, err, errlen);
}
int loom_hip_ciface_batch_matmul_f16(const loom_memref3_t* arg0, const loom_memref3_t* arg1,
                                     const loom_memref3_t* arg2, int64_t tile_b, int64_t tile_m,
                                     int64_t tile_n, int64_t tile_k, void* stream, char* err,
                                     size_t errlen) {
  const void* d[] = {arg0, arg1, arg2};
  Tiles t;
  t.t[LOOM_HIP_TILE_B] = tile_b, t.t[LOOM_HIP_TILE_M] = tile_m, t.t[LOOM_HIP_TILE_N] = tile_n;
  t.t[LOOM_HIP_TILE_K] = tile_k;
  return call("batch_matmul", true, d, 3, t.t, 0.f, 0, nullptr, 0, stream, err, errlen);
}

int loom_hip_ciface_split_k_matmul_gather(const loom_memref2_t* a, const loom_memref2_t* b,
                                          const loom_memref2_t* out, void* partials,
                                          size_t partials_bytes, int64_t tile_m, int64_t tile_n,
                                          int64_t tile_k, void* stream, char* err,
                                          size_t errlen) {
  const void* d[] = {a, b, out};
  Tiles t;
  t.t[LOOM_HIP_TILE_M] = tile_m, t.t[LOOM_HIP_TILE_N] = tile_n, t.t[LOOM_HIP_TILE_K] = tile_k;
  return call("split_k_matmul_gather", false, d, 3, t.t, 0.f, 0, partials, partials_bytes, stream,
              err, errlen);
}
int loom_hip_ciface_split_k_matmul_gather_f16(const loom_memref2_t* a, const loom_memref2_t* b,
                                              const loom_memref2_t* out, void* partials,
                                              size_t partials_bytes, int64_t tile_m,
                                              int64_t tile_n, int64_t tile_k, void* stream,
                                              char* err, size_t errlen) {
  const void* d[] = {a, b, out};
  Tiles t;
  t.t[LOOM_HIP_TILE_M] = tile_m, t.t[LOOM_HIP_TILE_N] = tile_n, t.t[LOOM_HIP_TILE_K] = tile_k;
  return call("split_k_matmul_gather", true, d, 3, t.t, 0.f, 0, partials, partials_bytes, stream,
              err, errlen);
}

int loom_hip_ciface_attention(const loom_memref3_t* k, const loom_memref3_t* v,
                              const loom_memref3_t* q, const loom_memref3_t* out, float scale,
                              int causal, int64_t tile_b, int64_t tile_m, int64_t tile_n,
                              void* stream, char* err, size_t errlen) {
  const void* d[] = {k, v, q, out};
  Tiles t;
  t.t[LOOM_HIP_TILE_B] = tile_b, t.t[LOOM_HIP_TILE_M] = tile_m, t.t[LOOM_HIP_TILE_N] = tile_n;
  return call("attention", false, d, 4, t.t, scale, causal, nullptr, 0, stream, err, errlen);
}
int loom_hip_ciface_attention_f16(const loom_memref3_t* k, const loom_memref3_t* v,
                                  const loom_memref3_t* q, const loom_memref3_t* out, float scale,
                                  int causal, int64_t tile_b, int64_t tile_m, int64_t tile_n,
                                  void* stream, char* err, size_t errlen) {
  const void* d[] = {k, v, q, out};
  Tiles t;
  t.t[LOOM_HIP_TILE_B] = tile_b, t.t[LOOM_HIP_TILE_M] = tile_m, t.t[LOOM_HIP_TILE_N] = tile_n;
  return call("attention", true, d, 4, t.t, scale, causal, nullptr, 0, stream, err, errlen);
}

int loom_hip_ciface_flash_decode(const loom_memref3_t* k, const loom_memref3_t* v,
                                 const loom_memref3_t* q, const loom_memref3_t* out,
                                 void* workspace, size_t workspace_bytes, float scale,
                                 int64_t tile_b, int64_t tile_s, int64_t tile_n, void* stream,
                                 char* err, size_t errlen) {
  const void* d[] = {k, v, q, out};
  Tiles t;
  t.t[LOOM_HIP_TILE_B] = tile_b, t.t[LOOM_HIP_TILE_S] = tile_s, t.t[LOOM_HIP_TILE_N] = tile_n;
  return call("flash_decode", false, d, 4, t.t, scale, 0, workspace, workspace_bytes, stream, err,
              errlen);
}
int loom_hip_ciface_flash_decode_f16(const loom_memref3_t* k, const loom_memref3_t* v,
                                     const loom_memref3_t* q, const loom_memref3_t* out,
                                     void* workspace, size_t workspace_bytes, float scale,
                                     int64_t tile_b, int64_t tile_s, int64_t tile_n, void* stream,
                                     char* err, size_t errlen) {
  const void* d[] = {k, v, q, out};
  Tiles t;
  t.t[LOOM_HIP_TILE_B] = tile_b, t.t[LOOM_HIP_TILE_S] = tile_s, t.t[LOOM_HIP_TILE_N] = tile_n;
  return call("flash_decode", true, d, 4, t.t, scale, 0, workspace, workspace_bytes, stream, err,
              errlen);
}

int loom_hip_ciface_helion_mamba2_chunk_scan_kernel(
    const loom_memref5_t* cb, const loom_memref4_t* x, const loom_memref4_t* dt,
    const loom_memref4_t* dA_cumsum, const loom_memref4_t* C, const loom_memref1_t* D,
    const loom_memref5_t* prev_states_T, const loom_memref4_t* out, int64_t tile_b,
    int64_t tile_h, int64_t tile_c, int64_t tile_m, int64_t tile_n, int64_t tile_k, void* stream,
    char* err, size_t errlen) {
  const void* d[] = {cb, x, dt, dA_cumsum, C, D, prev_states_T, out};
  Tiles t;
  t.t[LOOM_HIP_TILE_B] = tile_b, t.t[LOOM_HIP_TILE_H] = tile_h, t.t[LOOM_HIP_TILE_C] = tile_c;
  t.t[LOOM_HIP_TILE_M] = tile_m, t.t[LOOM_HIP_TILE_N] = tile_n, t.t[LOOM_HIP_TILE_K] = tile_k;
  return call("helion_mamba2_chunk_scan_kernel", false, d, 8, t.t, 0.f, 0, nullptr, 0, stream,
              err, errlen);
}
int loom_hip_ciface_helion_mamba2_chunk_scan_kernel_f16(
    const loom_memref5_t* cb, const loom_memref4_t* x, const loom_memref4_t* dt,
    const loom_memref4_t* dA_cumsum, const loom_memref4_t* C, const loom_memref1_t* D,
    const loom_memref5_t* prev_states_T, const loom_memref4_t* out, int64_t tile_b,
    int64_t tile_h, int64_t tile_c, int64_t tile_m, int64_t tile_n, int64_t tile_k, void* stream,
    char* err, size_t errlen) {
  const void* d[] = {cb, x, dt, dA_cumsum, C, D, prev_states_T, out};
  Tiles t;
  t.t[LOOM_HIP_TILE_B] = tile_b, t.t[LOOM_HIP_TILE_H] = tile_h, t.t[LOOM_HIP_TILE_C] = tile_c;
  t.t[LOOM_HIP_TILE_M] = tile_m, t.t[LOOM_HIP_TILE_N] = tile_n, t.t[LOOM_HIP_TILE_K] = tile_k;
  return call("helion_mamba2_chunk_scan_kernel", true, d, 8, t.t, 0.f, 0, nullptr, 0, stream, err,
              errlen);
}

int loom_hip_dispatch_memref(const char* variant, const void* const* descs, int ndescs,
                             float scale, int causal, void* workspace, size_t workspace_bytes,
                             void* stream, char* err, size_t errlen) {
  return dispatch_memref(variant, descs, ndescs, false, scale, causal, workspace, workspace_bytes,
                         stream, err, errlen);
}
int loom_hip_dispatch_memref_f16(const char* variant, const void* const* descs, int ndescs,
                                 float scale, int causal, void* workspace, size_t workspace_bytes,
                                 void* stream, char* err, size_t errlen) {
  return dispatch_memref(variant, descs, ndescs, true, scale, causal, workspace, workspace_bytes,
                         stream, err, errlen);
}

int loom_hip_check_memref(const char* variant, const void* const* descs, int ndescs, int f16,
                          float scale, char* err, size_t errlen) {
  bool& vo = loom_validate_only_flag();
  const bool outer = vo;
  vo = true;
  // a stand-in workspace of any size: only its presence is checked here
  void* ws = reinterpret_cast<void*>(uintptr_t(1) << 20);
  const int rc = dispatch_memref(variant, descs, ndescs, f16 != 0, scale, 0, ws, ~(size_t)0,
                                 nullptr, err, errlen);
  vo = outer;
  return rc;
}

}  // extern "C"
