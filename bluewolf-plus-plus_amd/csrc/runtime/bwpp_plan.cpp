// Launch-plan executor of libbwpp_hip.
//
// A launch plan is the lowered form of a BW++ graph (graph_ir.h:36-56 ops,
// after autodiff and fusion): named tensors with shapes over bound
// dimensions, and an ordered list of operator launches on them.  The
// executor parses it, builds the memory plan (liveness-based reuse of
// device buffers, as compiler/mem_plan.c:43-146 does for its symbolic
// buffers, but with byte sizes from the bound dims and without ever handing
// an operator's output the buffer of one of its own inputs), places every
// buffer in one device arena, and runs the launches through the C ABI on
// the handle's stream.
//
// Text format (one statement per line, '#' starts a comment):
//   bwpp.plan 1
//   dim NAME EXPR                     EXPR: product of integers / dims, e.g. B*T
//   value NAME f32 [EXPR,...] KIND    KIND: input | param | temp | output | const=<float>
//   view NAME of=BASE offset=EXPR ld=EXPR shape=[EXPR,EXPR]
//   op KIND out=A[,B..] in=X[,Y..] [key=value ...]
// Op kinds: matmul (ta, tb, epi, fuse), softmax, rmsnorm, layernorm,
// add / sub / mul / div / copy / silu (bcast; copy may take up to 4
// in/out pairs, one launch), reduce_sum, reduce_max,
// reduce_max_mask (axis), mean_square, silu_grad, softmax_grad,
// rmsnorm_grad, attention, attention_grad (batch, heads, causal, scale,
// layout).
// Tensors are row-major; row operators see [rows, cols] with cols the last
// dim and rows the product of the others; a view is a 2-D strided window
// (offset and row stride ld in elements) into another tensor's storage.
#include "bwpp_hip.h"
#include "internal.h"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

namespace {

enum class Kind { kInput, kParam, kTemp, kOutput, kConst, kView };

struct Value {
  std::string name;
  Kind kind = Kind::kTemp;
  std::vector<uint64_t> dims;
  std::vector<std::string> dim_text;
  uint32_t dtype = BWPP_HIP_F32;
  float const_value = 0.0f;
  // view
  int base = -1;
  uint64_t offset = 0, ld = 0;
  // placement
  int buffer = -1;  // memory-plan buffer (temps, outputs, consts)
  void *ptr = nullptr;
  int first_def = -1, last_use = -1;

  uint64_t elems() const {
    uint64_t n = 1;
    for (uint64_t d : dims) n *= d;
    return n;
  }
  uint64_t cols() const { return dims.empty() ? 1 : dims.back(); }
  uint64_t rows() const { return dims.empty() ? 1 : elems() / (cols() ? cols() : 1); }
  uint64_t row_stride() const { return kind == Kind::kView ? ld : cols(); }
};

struct Op {
  std::string kind;
  std::vector<int> outs, ins;
  std::map<std::string, std::string> attrs;
  int line = 0;
};

struct Buffer {
  uint64_t bytes = 0;
  size_t offset = 0;
  uint32_t dtype = BWPP_HIP_F32;
  std::vector<uint64_t> dims;
  std::vector<std::string> dim_text;
};

std::string trim(const std::string &s) {
  size_t a = s.find_first_not_of(" \t\r\n"), b = s.find_last_not_of(" \t\r\n");
  return a == std::string::npos ? std::string() : s.substr(a, b - a + 1);
}

std::vector<std::string> split(const std::string &s, char sep) {
  std::vector<std::string> out;
  std::string cur;
  for (char c : s) {
    if (c == sep) {
      out.push_back(trim(cur));
      cur.clear();
    } else {
      cur += c;
    }
  }
  out.push_back(trim(cur));
  return out;
}

}  // namespace

struct BwppHipPlan {
  BwppHip *h = nullptr;
  std::map<std::string, uint64_t> dims;
  std::vector<Value> values;
  std::map<std::string, int> by_name;
  std::vector<Op> ops;
  std::vector<Buffer> buffers;
  size_t arena_bytes = 0;
  BwppHipArena arena{};
  bool allocated = false;
  bool check_only = false;  // run_op validates arguments and launches nothing
  std::string err;
  // bwpp_hip_plan_capture: one run recorded as a HIP graph, and the
  // handle's workspace address its kernels were recorded with
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  const void *graph_ws = nullptr;
};

namespace {

BwppHipStatus perr(BwppHipPlan *p, BwppHipStatus st, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (p) p->err = buf;
  return st;
}

bool eval_expr(const BwppHipPlan &p, const std::string &e, uint64_t &out) {
  out = 1;
  for (const std::string &t : split(e, '*')) {
    if (t.empty()) return false;
    char *end = nullptr;
    unsigned long long v = strtoull(t.c_str(), &end, 10);
    if (end && *end == '\0') {
      out *= v;
    } else {
      auto it = p.dims.find(t);
      if (it == p.dims.end()) return false;
      out *= it->second;
    }
  }
  return true;
}

bool parse_kv(const std::string &tok, std::string &k, std::string &v) {
  size_t eq = tok.find('=');
  if (eq == std::string::npos) return false;
  k = tok.substr(0, eq);
  v = tok.substr(eq + 1);
  return true;
}

// Whitespace-separated tokens; [...] groups stay one token.
std::vector<std::string> tokens(const std::string &line) {
  std::vector<std::string> out;
  std::string cur;
  int depth = 0;
  for (char c : line) {
    if (c == '[') depth++;
    if (c == ']') depth--;
    if ((c == ' ' || c == '\t') && depth == 0) {
      if (!cur.empty()) out.push_back(cur);
      cur.clear();
    } else {
      cur += c;
    }
  }
  if (!cur.empty()) out.push_back(cur);
  return out;
}

BwppHipStatus parse_dims(BwppHipPlan &p, const std::string &tok, Value &v, int ln) {
  if (tok.size() < 2 || tok.front() != '[' || tok.back() != ']')
    return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: shape must be [d0,d1,...]", ln);
  const std::string inner = tok.substr(1, tok.size() - 2);
  if (trim(inner).empty()) return BWPP_HIP_OK;
  for (const std::string &d : split(inner, ',')) {
    uint64_t n = 0;
    if (!eval_expr(p, d, n)) return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: unknown dim '%s'", ln, d.c_str());
    v.dims.push_back(n);
    v.dim_text.push_back(d);
  }
  if (v.dims.size() > 4) return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: rank above 4", ln);
  return BWPP_HIP_OK;
}

BwppHipStatus parse(BwppHipPlan &p, const char *text) {
  std::istringstream in(text);
  std::string raw;
  int ln = 0;
  bool header = false;
  while (std::getline(in, raw)) {
    ++ln;
    std::string line = raw.substr(0, raw.find('#'));
    line = trim(line);
    if (line.empty()) continue;
    std::vector<std::string> t = tokens(line);
    if (!header) {
      if (t.size() != 2 || t[0] != "bwpp.plan" || t[1] != "1")
        return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: expected 'bwpp.plan 1'", ln);
      header = true;
      continue;
    }
    if (t[0] == "dim") {
      uint64_t n = 0;
      if (t.size() != 3 || !eval_expr(p, t[2], n))
        return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: bad dim", ln);
      p.dims[t[1]] = n;
    } else if (t[0] == "value") {
      if (t.size() != 5) return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: value NAME DTYPE [dims] KIND", ln);
      if (p.by_name.count(t[1])) return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: '%s' redefined", ln, t[1].c_str());
      Value v;
      v.name = t[1];
      if (t[2] == "f32") v.dtype = BWPP_HIP_F32;
      else if (t[2] == "bf16") v.dtype = BWPP_HIP_BF16;
      else return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: dtype f32 or bf16", ln);
      BwppHipStatus s = parse_dims(p, t[3], v, ln);
      if (s != BWPP_HIP_OK) return s;
      const std::string &k = t[4];
      if (k == "input") v.kind = Kind::kInput;
      else if (k == "param") v.kind = Kind::kParam;
      else if (k == "temp") v.kind = Kind::kTemp;
      else if (k == "output") v.kind = Kind::kOutput;
      else if (k.rfind("const=", 0) == 0) {
        // const=NUM or const=NUM/EXPR (e.g. 1/B*T*D for a mean)
        v.kind = Kind::kConst;
        const std::string c = k.substr(6);
        const size_t slash = c.find('/');
        v.const_value = strtof(c.substr(0, slash).c_str(), nullptr);
        if (slash != std::string::npos) {
          uint64_t den = 0;
          if (!eval_expr(p, c.substr(slash + 1), den) || den == 0)
            return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: bad const divisor", ln);
          v.const_value = (float)((double)v.const_value / (double)den);
        }
        if (v.dtype != BWPP_HIP_F32) return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: const must be f32", ln);
      } else {
        return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: unknown kind '%s'", ln, k.c_str());
      }
      p.by_name[v.name] = (int)p.values.size();
      p.values.push_back(v);
    } else if (t[0] == "view") {
      if (t.size() < 2) return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: view NAME ...", ln);
      Value v;
      v.name = t[1];
      v.kind = Kind::kView;
      for (size_t i = 2; i < t.size(); ++i) {
        std::string k, val;
        if (!parse_kv(t[i], k, val)) return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: bad '%s'", ln, t[i].c_str());
        if (k == "of") {
          auto it = p.by_name.find(val);
          if (it == p.by_name.end() || p.values[it->second].kind == Kind::kView)
            return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: view of unknown or view '%s'", ln, val.c_str());
          v.base = it->second;
        } else if (k == "offset" || k == "ld") {
          uint64_t n = 0;
          if (!eval_expr(p, val, n)) return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: bad %s", ln, k.c_str());
          (k == "offset" ? v.offset : v.ld) = n;
        } else if (k == "shape") {
          BwppHipStatus s = parse_dims(p, val, v, ln);
          if (s != BWPP_HIP_OK) return s;
        } else {
          return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: unknown view key '%s'", ln, k.c_str());
        }
      }
      if (v.base < 0 || v.dims.size() != 2 || v.ld < v.dims[1])
        return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: view needs of=, 2-D shape=, ld >= cols", ln);
      const Value &b = p.values[v.base];
      v.dtype = b.dtype;
      if (v.offset + (v.dims[0] - 1) * v.ld + v.dims[1] > b.elems())
        return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: view '%s' runs past '%s'", ln, v.name.c_str(),
                    b.name.c_str());
      p.by_name[v.name] = (int)p.values.size();
      p.values.push_back(v);
    } else if (t[0] == "op") {
      if (t.size() < 2) return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: op KIND ...", ln);
      Op op;
      op.kind = t[1];
      op.line = ln;
      for (size_t i = 2; i < t.size(); ++i) {
        std::string k, val;
        if (!parse_kv(t[i], k, val)) return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: bad '%s'", ln, t[i].c_str());
        if (k == "out" || k == "in") {
          for (const std::string &n : split(val, ',')) {
            auto it = p.by_name.find(n);
            if (it == p.by_name.end())
              return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: unknown value '%s'", ln, n.c_str());
            (k == "out" ? op.outs : op.ins).push_back(it->second);
          }
        } else {
          op.attrs[k] = val;
        }
      }
      if (op.outs.empty()) return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: op without out=", ln);
      p.ops.push_back(op);
    } else {
      return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d: unknown statement '%s'", ln, t[0].c_str());
    }
  }
  if (!header) return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "empty plan");
  return BWPP_HIP_OK;
}

// Storage owner of a value (a view's base, else itself).
int owner(const BwppHipPlan &p, int v) { return p.values[v].kind == Kind::kView ? p.values[v].base : v; }

bool planned(Kind k) { return k == Kind::kTemp || k == Kind::kOutput || k == Kind::kConst; }

// Liveness and buffer assignment.  A buffer is released after the last op
// that reads its value, and only after that op's outputs got buffers, so no
// op ever writes into the storage of one of its own inputs (the reference
// planner frees first, mem_plan.c:89-140).  Outputs and consts keep their
// buffers; temps reuse a released buffer of the same dtype and byte size.
BwppHipStatus plan_memory(BwppHipPlan &p) {
  const int nops = (int)p.ops.size();
  std::vector<int> first_read(p.values.size(), -1);
  for (int i = 0; i < nops; ++i) {
    for (int v : p.ops[i].ins) {
      const int oi = owner(p, v);
      Value &o = p.values[oi];
      o.last_use = i;
      if (first_read[oi] < 0) first_read[oi] = i;
    }
    for (int v : p.ops[i].outs) {
      Value &o = p.values[owner(p, v)];
      if (o.first_def < 0) o.first_def = i;
      if (o.last_use < i) o.last_use = i;
    }
  }
  for (Value &v : p.values)
    if (v.kind == Kind::kOutput || v.kind == Kind::kConst) v.last_use = nops;
  for (int i = 0; i < (int)p.values.size(); ++i) {
    const Value &v = p.values[i];
    if (v.kind == Kind::kTemp && v.first_def < 0 && v.last_use >= 0)
      return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "'%s' is read but never written", v.name.c_str());
    if ((v.kind == Kind::kTemp || v.kind == Kind::kOutput) && first_read[i] >= 0 && first_read[i] < v.first_def)
      return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "'%s' is read (line %d) before it is written", v.name.c_str(),
                  p.ops[first_read[i]].line);
  }
  std::vector<int> free_list;
  auto bytes_of = [](const Value &v) { return v.elems() * (v.dtype == BWPP_HIP_BF16 ? 2 : 4); };
  auto take = [&](int vi) {
    Value &v = p.values[vi];
    if (v.buffer >= 0) return;
    const uint64_t nb = bytes_of(v);
    for (size_t f = 0; f < free_list.size(); ++f) {
      Buffer &b = p.buffers[free_list[f]];
      if (b.bytes == nb && b.dtype == v.dtype && v.kind == Kind::kTemp) {
        v.buffer = free_list[f];
        free_list.erase(free_list.begin() + f);
        return;
      }
    }
    Buffer b;
    b.bytes = nb;
    b.dtype = v.dtype;
    b.dims = v.dims;
    b.dim_text = v.dim_text;
    v.buffer = (int)p.buffers.size();
    p.buffers.push_back(b);
  };
  for (int i = 0; i < (int)p.values.size(); ++i)
    if (p.values[i].kind == Kind::kConst) take(i);
  for (int i = 0; i < nops; ++i) {
    for (int v : p.ops[i].outs) {
      const int o = owner(p, v);
      if (planned(p.values[o].kind)) take(o);
    }
    // Release temps whose last use is this op: inputs read for the last
    // time, and outputs nothing reads later (after this op's outputs have
    // their buffers, so none of them shares a buffer with its own inputs).
    for (const std::vector<int> *list : {&p.ops[i].ins, &p.ops[i].outs})
      for (int v : *list) {
        const int o = owner(p, v);
        Value &val = p.values[o];
        if (val.kind == Kind::kTemp && val.last_use == i && val.buffer >= 0 &&
            std::find(free_list.begin(), free_list.end(), val.buffer) == free_list.end())
          free_list.push_back(val.buffer);
      }
  }
  size_t off = 0;
  for (Buffer &b : p.buffers) {
    off = (off + 255) & ~(size_t)255;
    b.offset = off;
    off += b.bytes;
  }
  p.arena_bytes = off;
  return BWPP_HIP_OK;
}

}  // namespace

namespace {
BwppHipStatus run_op(BwppHipPlan &p, const Op &op);
}  // namespace

extern "C" BwppHipStatus bwpp_hip_plan_create(BwppHip *h, const char *text, BwppHipPlan **out) {
  if (!out) return BWPP_HIP_ERR_INVALID_ARG;
  *out = nullptr;
  if (!text) return BWPP_HIP_ERR_INVALID_ARG;
  BwppHipPlan *p = new BwppHipPlan();
  p->h = h;
  BwppHipStatus s = parse(*p, text);
  if (s == BWPP_HIP_OK) s = plan_memory(*p);
  // Every op checks its arguments once here, so a bad plan fails at creation.
  p->check_only = true;
  for (size_t i = 0; s == BWPP_HIP_OK && i < p->ops.size(); ++i) s = run_op(*p, p->ops[i]);
  p->check_only = false;
  *out = p;  // returned even on failure so that the caller can read the error
  return s;
}

namespace {
void drop_graph(BwppHipPlan *p) {
  if (p->exec) (void)hipGraphExecDestroy(p->exec);
  if (p->graph) (void)hipGraphDestroy(p->graph);
  p->exec = nullptr;
  p->graph = nullptr;
}
}  // namespace

extern "C" void bwpp_hip_plan_destroy(BwppHipPlan *p) {
  if (!p) return;
  drop_graph(p);
  if (p->allocated) bwpp_hip_arena_destroy(&p->arena);
  delete p;
}

extern "C" BwppHipStatus bwpp_hip_plan_capture(BwppHipPlan *p) {
  if (!p) return BWPP_HIP_ERR_INVALID_ARG;
  drop_graph(p);
  if (!p->h) return perr(p, BWPP_HIP_ERR_INVALID_ARG, "plan created without a device handle");
  hipStream_t st = static_cast<hipStream_t>(bwpp_hip_get_stream(p->h));
  if (!st) return perr(p, BWPP_HIP_ERR_UNSUPPORTED, "capture needs a non-default stream on the handle");
  // One eager run first: every workspace the ops use reaches its final size,
  // so nothing allocates while the stream is being captured.
  BwppHipStatus s = bwpp_hip_plan_run(p);
  if (s != BWPP_HIP_OK) return s;
  if (hipStreamSynchronize(st) != hipSuccess) return perr(p, BWPP_HIP_ERR_HIP, "stream synchronize failed");
  hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return perr(p, BWPP_HIP_ERR_HIP, "hipStreamBeginCapture: %s", hipGetErrorString(e));
  for (const Op &op : p->ops) {
    s = run_op(*p, op);
    if (s != BWPP_HIP_OK) break;
  }
  hipGraph_t g = nullptr;
  e = hipStreamEndCapture(st, &g);
  if (s != BWPP_HIP_OK) {
    if (g) (void)hipGraphDestroy(g);
    return s;
  }
  if (e != hipSuccess || !g) return perr(p, BWPP_HIP_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
  p->graph = g;
  e = hipGraphInstantiate(&p->exec, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    drop_graph(p);
    return perr(p, BWPP_HIP_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
  }
  p->graph_ws = bwpp_hip_workspace(p->h);
  return BWPP_HIP_OK;
}

extern "C" BwppHipStatus bwpp_hip_plan_replay(BwppHipPlan *p) {
  if (!p) return BWPP_HIP_ERR_INVALID_ARG;
  if (!p->exec) return perr(p, BWPP_HIP_ERR_INVALID_ARG, "no captured graph (capture after the last bind)");
  // An op on the handle that needed a larger workspace freed the one the
  // graph's kernels address: refuse rather than replay into freed memory.
  if (bwpp_hip_workspace(p->h) != p->graph_ws)
    return perr(p, BWPP_HIP_ERR_INVALID_ARG,
                "the handle's workspace was reallocated after capture (a larger op ran on it): capture again");
  hipStream_t st = static_cast<hipStream_t>(bwpp_hip_get_stream(p->h));
  hipError_t e = hipGraphLaunch(p->exec, st);
  if (e != hipSuccess) return perr(p, BWPP_HIP_ERR_HIP, "hipGraphLaunch: %s", hipGetErrorString(e));
  return BWPP_HIP_OK;
}

extern "C" const char *bwpp_hip_plan_last_error(const BwppHipPlan *p) { return p ? p->err.c_str() : ""; }

extern "C" size_t bwpp_hip_plan_arena_bytes(const BwppHipPlan *p) { return p ? p->arena_bytes : 0; }

extern "C" BwppHipStatus bwpp_hip_plan_allocate(BwppHipPlan *p) {
  if (!p) return BWPP_HIP_ERR_INVALID_ARG;
  if (!p->h) return perr(p, BWPP_HIP_ERR_INVALID_ARG, "plan created without a device handle");
  if (p->allocated) return BWPP_HIP_OK;
  BwppHipStatus s = bwpp_hip_arena_init(p->h, &p->arena, p->arena_bytes ? p->arena_bytes : 256);
  if (s != BWPP_HIP_OK) return perr(p, s, "arena: %s", bwpp_hip_last_error(p->h));
  // The arena places buffers at their planned offsets (one bump allocation).
  if (!bwpp_hip_arena_alloc(&p->arena, p->arena_bytes ? p->arena_bytes : 1, 256))
    return perr(p, BWPP_HIP_ERR_OUT_OF_MEMORY, "arena too small");
  p->allocated = true;
  for (Value &v : p->values)
    if (planned(v.kind)) v.ptr = p->arena.buffer + p->buffers[v.buffer].offset;
  for (Value &v : p->values) {
    if (v.kind != Kind::kConst) continue;
    std::vector<float> host(v.elems(), v.const_value);
    s = bwpp_hip_copy_to_device(p->h, v.ptr, host.data(), host.size() * sizeof(float));
    if (s != BWPP_HIP_OK) return perr(p, s, "const '%s': %s", v.name.c_str(), bwpp_hip_last_error(p->h));
  }
  return BWPP_HIP_OK;
}

extern "C" BwppHipStatus bwpp_hip_plan_bind(BwppHipPlan *p, const char *name, void *ptr) {
  if (!p || !name) return BWPP_HIP_ERR_INVALID_ARG;
  auto it = p->by_name.find(name);
  if (it == p->by_name.end()) return perr(p, BWPP_HIP_ERR_INVALID_ARG, "no value '%s'", name);
  Value &v = p->values[it->second];
  if (v.kind != Kind::kInput && v.kind != Kind::kParam)
    return perr(p, BWPP_HIP_ERR_INVALID_ARG, "'%s' is not an input or param", name);
  if (v.ptr != ptr) drop_graph(p);  // the graph holds the old address
  v.ptr = ptr;
  return BWPP_HIP_OK;
}

extern "C" void *bwpp_hip_plan_value_ptr(const BwppHipPlan *p, const char *name) {
  if (!p || !name) return nullptr;
  auto it = p->by_name.find(name);
  if (it == p->by_name.end()) return nullptr;
  const Value &v = p->values[it->second];
  if (v.kind == Kind::kView) {
    const Value &b = p->values[v.base];
    if (!b.ptr) return nullptr;
    return static_cast<unsigned char *>(b.ptr) + v.offset * (v.dtype == BWPP_HIP_BF16 ? 2 : 4);
  }
  return v.ptr;
}

namespace {

const char *dtype_name(uint32_t dt) { return dt == BWPP_HIP_BF16 ? "bf16" : "f32"; }

std::string attr(const Op &op, const char *k, const char *dflt) {
  auto it = op.attrs.find(k);
  return it == op.attrs.end() ? std::string(dflt) : it->second;
}

// In check-only mode (plan creation) each op validates its arguments and
// shapes and launches nothing.
#define BWPP_PLAN_CALL(expr) (p.check_only ? BWPP_HIP_OK : (expr))

BwppHipStatus run_op(BwppHipPlan &p, const Op &op) {
  BwppHip *h = p.h;
  auto val = [&](int i) -> const Value & { return p.values[i]; };
  auto ptr = [&](int i) { return bwpp_hip_plan_value_ptr(&p, p.values[i].name.c_str()); };
  auto need = [&](size_t nin, size_t nout) {
    return op.ins.size() >= nin && op.outs.size() >= nout;
  };
  auto bad = [&](const char *what) {
    return perr(&p, BWPP_HIP_ERR_INVALID_ARG, "line %d (%s): %s", op.line, op.kind.c_str(), what);
  };
  auto f32 = [&](int i) { return static_cast<float *>(ptr(i)); };
  auto num = [&](const char *k, double dflt) {
    auto it = op.attrs.find(k);
    if (it == op.attrs.end()) return dflt;
    uint64_t n = 0;
    if (eval_expr(p, it->second, n) && it->second.find('.') == std::string::npos) return (double)n;
    return strtod(it->second.c_str(), nullptr);
  };
  const std::string &k = op.kind;
  BwppHipStatus s = BWPP_HIP_OK;
  // dtypes: matmul and attention take f32 or bf16 operands of one dtype
  // (lse is f32); every other operator is f32 only.
  {
    auto dt = [&](int i) { return val(i).dtype; };
    if (k == "matmul" || k == "attention" || k == "attention_grad") {
      const uint32_t d0 = dt(op.ins[0]);
      const bool att = k != "matmul";
      for (size_t j = 0; j < op.ins.size(); ++j)
        if (!(k == "attention_grad" && j == 5) && dt(op.ins[j]) != d0) return bad("operands of different dtypes");
      for (size_t j = 0; j < op.outs.size(); ++j) {
        const bool lse = att && k == "attention" && j == 1;
        if (dt(op.outs[j]) != (lse ? (uint32_t)BWPP_HIP_F32 : d0)) return bad("output dtype does not match");
      }
      if (k == "attention_grad" && op.ins.size() > 5 && dt(op.ins[5]) != BWPP_HIP_F32) return bad("lse must be f32");
    } else {
      for (const std::vector<int> *list : {&op.ins, &op.outs})
        for (int v : *list)
          if (dt(v) != BWPP_HIP_F32) return bad("this operator takes f32 values only");
    }
  }
  if (k == "matmul") {
    if (op.ins.size() < 2 || op.outs.empty()) return bad("in=A,B[,bias][,aux] out=C[,C2]");
    const Value &A = val(op.ins[0]), &B = val(op.ins[1]), &C = val(op.outs[0]);
    const uint32_t ta = (uint32_t)num("ta", 0), tb = (uint32_t)num("tb", 0);
    const uint64_t M = C.rows(), N = C.cols();
    const uint64_t K = ta ? A.rows() : A.cols();
    if ((ta ? A.cols() : A.rows()) != M || (tb ? B.cols() : B.rows()) != K || (tb ? B.rows() : B.cols()) != N)
      return bad("operand shapes do not match");
    const std::string e = attr(op, "epi", "none");
    if (e != "none" && e != "add" && e != "silu" && e != "add_silu")
      return bad("epi must be none, add, silu or add_silu");
    uint32_t epi = e == "add" ? BWPP_HIP_EPILOGUE_ADD : e == "silu" ? BWPP_HIP_EPILOGUE_SILU
                   : e == "add_silu" ? BWPP_HIP_EPILOGUE_ADD_SILU : BWPP_HIP_EPILOGUE_NONE;
    BwppMatmulParams mp = {(uint32_t)M, (uint32_t)N, (uint32_t)K, (uint32_t)A.row_stride(), (uint32_t)B.row_stride(),
                           (uint32_t)C.row_stride(), C.dtype, epi, ta, tb};
    // fuse=residual (C = epi(A.B) + aux), dual_silu (out=C,C2 with C2 =
    // SiLU(C)), silu_grad (C = A.B * silu'(aux)): the inputs are then
    // A, B, the bias when epi adds one, and aux.
    const std::string fz = attr(op, "fuse", "none");
    if (fz != "none" && fz != "residual" && fz != "dual_silu" && fz != "silu_grad")
      return bad("fuse must be none, residual, dual_silu or silu_grad");
    if (fz == "none") {
      if (op.ins.size() > 3 || op.outs.size() != 1) return bad("in=A,B[,bias] out=C");
      s = BWPP_PLAN_CALL(bwpp_hip_dispatch_matmul(h, ptr(op.ins[0]), ptr(op.ins[1]), ptr(op.outs[0]),
                                                  op.ins.size() > 2 ? ptr(op.ins[2]) : nullptr, mp));
    } else {
      BwppHipFusionParams fp = {};
      fp.kind = fz == "residual" ? BWPP_HIP_FUSE_RESIDUAL : fz == "dual_silu" ? BWPP_HIP_FUSE_DUAL_SILU
                                                                            : BWPP_HIP_FUSE_SILU_GRAD;
      const bool has_bias = (epi & BWPP_HIP_EPILOGUE_ADD) != 0, has_aux = fz != "dual_silu";
      const size_t nin = 2 + (has_bias ? 1 : 0) + (has_aux ? 1 : 0), nout = fz == "dual_silu" ? 2 : 1;
      if (op.ins.size() != nin || op.outs.size() != nout)
        return bad("fused matmul: in=A,B[,bias],aux (residual, silu_grad) or in=A,B[,bias] out=C,C2 (dual_silu)");
      const int ai = has_aux ? op.ins[nin - 1] : -1, c2i = nout == 2 ? op.outs[1] : -1;
      if (ai >= 0 && (val(ai).rows() != M || val(ai).cols() != N)) return bad("aux must have C's shape");
      if (c2i >= 0 && (val(c2i).rows() != M || val(c2i).cols() != N)) return bad("C2 must have C's shape");
      fp.ld_aux = ai >= 0 ? (uint32_t)val(ai).row_stride() : 0u;
      fp.ld_c2 = c2i >= 0 ? (uint32_t)val(c2i).row_stride() : 0u;
      s = BWPP_PLAN_CALL(bwpp_hip_dispatch_matmul_fused(h, ptr(op.ins[0]), ptr(op.ins[1]), ptr(op.outs[0]),
                                                        has_bias ? ptr(op.ins[2]) : nullptr,
                                                        ai >= 0 ? f32(ai) : nullptr, c2i >= 0 ? f32(c2i) : nullptr,
                                                        mp, fp));
    }
  } else if (k == "softmax" || k == "rmsnorm" || k == "layernorm") {
    if (!need(1, 1)) return bad("in=X[,gamma[,beta]] out=Y");
    const Value &X = val(op.ins[0]);
    const float eps = (float)num("eps", 1e-5);
    if (k == "softmax") {
      BwppSoftmaxParams sp = {(uint32_t)X.rows(), (uint32_t)X.cols(), (uint32_t)X.row_stride()};
      s = BWPP_PLAN_CALL(bwpp_hip_dispatch_softmax(h, f32(op.ins[0]), f32(op.outs[0]), sp));
    } else {
      BwppRmsnormParams rp = {(uint32_t)X.rows(), (uint32_t)X.cols(), (uint32_t)X.row_stride(), eps};
      const float *g = op.ins.size() > 1 ? f32(op.ins[1]) : nullptr;
      const float *bt = op.ins.size() > 2 ? f32(op.ins[2]) : nullptr;
      s = BWPP_PLAN_CALL(k == "rmsnorm" ? bwpp_hip_dispatch_rmsnorm(h, f32(op.ins[0]), g, bt, f32(op.outs[0]), rp)
                         : bwpp_hip_dispatch_layernorm(h, f32(op.ins[0]), g, bt, f32(op.outs[0]), rp));
    }
  } else if (k == "copy" && (op.ins.size() > 1 || op.outs.size() > 1)) {
    // several copies in one launch: pair i copies in[i] into out[i]
    // (full shapes, any row strides; at most 4 pairs)
    if (op.ins.size() != op.outs.size() || op.ins.size() > BWPP_COPY_MULTI_MAX)
      return bad("multi-pair copy: in=X1,..,Xn out=Y1,..,Yn with n <= 4");
    if (attr(op, "bcast", "full") != "full") return bad("multi-pair copy takes bcast=full");
    const float *src[BWPP_COPY_MULTI_MAX];
    float *dst[BWPP_COPY_MULTI_MAX];
    uint32_t lds[BWPP_COPY_MULTI_MAX], ldd[BWPP_COPY_MULTI_MAX], rows[BWPP_COPY_MULTI_MAX], cols[BWPP_COPY_MULTI_MAX];
    const uint32_t n = (uint32_t)op.ins.size();
    for (uint32_t i = 0; i < n; ++i) {
      const Value &X = val(op.ins[i]), &Y = val(op.outs[i]);
      if (X.rows() != Y.rows() || X.cols() != Y.cols()) return bad("copy needs equal shapes");
      src[i] = f32(op.ins[i]);
      dst[i] = f32(op.outs[i]);
      lds[i] = (uint32_t)X.row_stride();
      ldd[i] = (uint32_t)Y.row_stride();
      rows[i] = (uint32_t)Y.rows();
      cols[i] = (uint32_t)Y.cols();
    }
    s = BWPP_PLAN_CALL(bwpp_hip_copy_strided_multi(h, n, src, lds, dst, ldd, rows, cols));
  } else if (k == "add" || k == "sub" || k == "mul" || k == "div" || k == "copy" || k == "silu") {
    const bool unary = k == "copy" || k == "silu";
    if (!need(unary ? 1 : 2, 1)) return bad("in=A,B (or in=B for copy / silu) out=C");
    const Value &C = val(op.outs[0]);
    const int bi = op.ins[unary ? 0 : 1];
    const std::string bm = attr(op, "bcast", "full");
    if (bm != "full" && bm != "row" && bm != "col" && bm != "scalar")
      return bad("bcast must be full, row, col or scalar");
    const uint32_t bmode = bm == "row" ? BWPP_HIP_BCAST_ROW : bm == "col" ? BWPP_HIP_BCAST_COL
                           : bm == "scalar" ? BWPP_HIP_BCAST_SCALAR : BWPP_HIP_BCAST_FULL;
    const uint32_t opc = k == "add" ? BWPP_HIP_OP_ADD : k == "sub" ? BWPP_HIP_OP_SUB : k == "mul" ? BWPP_HIP_OP_MUL
                         : k == "div" ? BWPP_HIP_OP_DIV : k == "copy" ? BWPP_HIP_OP_COPY : BWPP_HIP_OP_SILU;
    if (k == "copy" && bmode == BWPP_HIP_BCAST_FULL && val(bi).row_stride() != C.row_stride()) {
      // a copy between a tensor and a strided view (e.g. one weight into
      // its column block of a concatenation): strides may differ
      const Value &X = val(bi);
      if (X.rows() != C.rows() || X.cols() != C.cols()) return bad("copy needs equal shapes");
      s = BWPP_PLAN_CALL(bwpp_hip_copy_strided(h, f32(bi), (uint32_t)X.row_stride(), f32(op.outs[0]),
                                               (uint32_t)C.row_stride(), (uint32_t)C.rows(), (uint32_t)C.cols()));
      if (s != BWPP_HIP_OK) return perr(&p, s, "line %d (%s): %s", op.line, k.c_str(), bwpp_hip_last_error(h));
      return BWPP_HIP_OK;
    }
    if (bmode == BWPP_HIP_BCAST_FULL && val(bi).row_stride() != C.row_stride()) return bad("full b needs C's stride");
    if (!unary && val(op.ins[0]).row_stride() != C.row_stride()) return bad("a needs C's stride");
    BwppElementwiseParams ep = {(uint32_t)C.rows(), (uint32_t)C.cols(), (uint32_t)C.row_stride(), opc, bmode};
    s = BWPP_PLAN_CALL(
        bwpp_hip_dispatch_elementwise(h, unary ? nullptr : f32(op.ins[0]), f32(bi), f32(op.outs[0]), ep));
  } else if (k == "reduce_sum") {
    if (!need(1, 1)) return bad("in=X out=Y");
    const Value &X = val(op.ins[0]);
    BwppReduceParams rp = {(uint32_t)X.rows(), (uint32_t)X.cols(), (uint32_t)X.row_stride(),
                           (int32_t)num("axis", 1)};
    s = BWPP_PLAN_CALL(bwpp_hip_dispatch_reduce_sum(h, f32(op.ins[0]), f32(op.outs[0]), rp));
  } else if (k == "mean_square") {
    // loss = loss_scale * sum(X^2) (one element) and dX = grad_scale * X;
    // the scales are one-element values (consts), absent = 1.
    if (!need(1, 1) || op.ins.size() > 3 || op.outs.size() > 2)
      return bad("in=X[,loss_scale[,grad_scale]] out=loss[,dX]");
    const Value &X = val(op.ins[0]);
    if (val(op.outs[0]).elems() != 1) return bad("mean_square: loss must have one element");
    if (op.outs.size() > 1 && (val(op.outs[1]).elems() != X.elems() || val(op.outs[1]).row_stride() != X.row_stride()))
      return bad("mean_square: dX must have X's shape and row stride");
    for (size_t i = 1; i < op.ins.size(); ++i)
      if (val(op.ins[i]).elems() != 1) return bad("mean_square: scales must have one element");
    BwppMeanSquareParams mp = {(uint32_t)X.rows(), (uint32_t)X.cols(), (uint32_t)X.row_stride()};
    s = BWPP_PLAN_CALL(bwpp_hip_dispatch_mean_square(h, f32(op.ins[0]), op.ins.size() > 1 ? f32(op.ins[1]) : nullptr,
                                                     op.ins.size() > 2 ? f32(op.ins[2]) : nullptr, f32(op.outs[0]),
                                                     op.outs.size() > 1 ? f32(op.outs[1]) : nullptr, mp));
  } else if (k == "reduce_max" || k == "reduce_max_mask") {
    // Graph ops BWPP_GOP_REDUCE_MAX (values; graph_ir.c:663-695) and
    // BWPP_GOP_REDUCE_MAX_MASK (bwpp_cpu_ref.c:146-190) along `axis`.
    if (!need(1, 1)) return bad("in=X out=Y");
    const Value &X = val(op.ins[0]);
    BwppReduceParams rp = {(uint32_t)X.rows(), (uint32_t)X.cols(), (uint32_t)X.row_stride(),
                           (int32_t)num("axis", 1)};
    const uint64_t want = k == "reduce_max_mask" ? X.rows() * X.cols() : rp.axis == 0 ? X.cols() : X.rows();
    if (val(op.outs[0]).elems() != want) return bad("output size does not match the reduction");
    if (k == "reduce_max_mask" && val(op.outs[0]).row_stride() != X.row_stride())
      return bad("mask needs X's row stride");
    s = BWPP_PLAN_CALL(k == "reduce_max"
                           ? bwpp_hip_dispatch_reduce_max(h, f32(op.ins[0]), f32(op.outs[0]), nullptr, rp)
                           : bwpp_hip_dispatch_reduce_max_mask(h, f32(op.ins[0]), f32(op.outs[0]), rp));
  } else if (k == "silu_grad") {
    if (!need(2, 1)) return bad("in=X,dY out=dX");
    s = BWPP_PLAN_CALL(
        bwpp_hip_dispatch_silu_grad(h, f32(op.ins[0]), f32(op.ins[1]), f32(op.outs[0]), val(op.ins[0]).elems()));
  } else if (k == "softmax_grad") {
    if (!need(2, 1)) return bad("in=Y,dY out=dX");
    const Value &Y = val(op.ins[0]);
    BwppSoftmaxParams sp = {(uint32_t)Y.rows(), (uint32_t)Y.cols(), (uint32_t)Y.row_stride()};
    s = BWPP_PLAN_CALL(bwpp_hip_dispatch_softmax_grad(h, f32(op.ins[0]), f32(op.ins[1]), f32(op.outs[0]), sp));
  } else if (k == "rmsnorm_grad") {
    // A fourth input is added to dX in the same pass (the residual branch's
    // gradient, dX = acc + rmsnorm_grad).
    if (!need(3, 1) || op.ins.size() > 4) return bad("in=X,gamma,dY[,acc] out=dX[,dgamma[,dbeta]]");
    const Value &X = val(op.ins[0]);
    if (op.ins.size() > 3 && val(op.ins[3]).row_stride() != X.row_stride())
      return bad("rmsnorm_grad: acc must have the row stride of X");
    BwppRmsnormParams rp = {(uint32_t)X.rows(), (uint32_t)X.cols(), (uint32_t)X.row_stride(), (float)num("eps", 1e-5)};
    s = BWPP_PLAN_CALL(bwpp_hip_dispatch_rmsnorm_grad_acc(
        h, f32(op.ins[0]), f32(op.ins[1]), f32(op.ins[2]), op.ins.size() > 3 ? f32(op.ins[3]) : nullptr,
        f32(op.outs[0]), op.outs.size() > 1 ? f32(op.outs[1]) : nullptr, op.outs.size() > 2 ? f32(op.outs[2]) : nullptr,
        rp));
  } else if (k == "attention" || k == "attention_grad") {
    // q / k / v (and o, do, dq, dk, dv) are [batch*seq, heads*dim] row
    // blocks: head h of a row starts at column h*dim.
    const bool grad = k == "attention_grad";
    if (grad ? !need(6, 3) : !need(3, 1))
      return bad(grad ? "in=Q,K,V,O,dO,LSE out=dQ,dK,dV" : "in=Q,K,V out=O[,LSE]");
    // layout=bshd (default): [batch*seq, heads*dim] row blocks, head h of a
    // row at column h*dim.  layout=bhsd: [batch, heads, seq, dim] with one
    // row per (batch, head, position).
    const uint64_t B = (uint64_t)num("batch", 1), H = (uint64_t)num("heads", 1);
    const std::string lay = attr(op, "layout", "bshd");
    if (lay != "bshd" && lay != "bhsd") return bad("layout must be bshd or bhsd");
    const bool bhsd = lay == "bhsd";
    const Value &Q = val(op.ins[0]), &Kv = val(op.ins[1]), &V = val(op.ins[2]);
    const Value &O = grad ? val(op.ins[3]) : val(op.outs[0]);
    const uint64_t qs = bhsd ? B * H : B;  // row blocks per tensor
    if (!B || !H || Q.rows() % qs || Kv.rows() % qs || (!bhsd && (Q.cols() % H || V.cols() % H)))
      return bad("bad batch / heads");
    const uint64_t M = Q.rows() / qs, N = Kv.rows() / qs;
    const uint64_t dk = bhsd ? Q.cols() : Q.cols() / H, dv = bhsd ? V.cols() : V.cols() / H;
    BwppAttentionParams ap = {};
    ap.M = (uint32_t)M;
    ap.N = (uint32_t)N;
    ap.K = (uint32_t)dk;
    ap.D = (uint32_t)dv;
    ap.ldq = (uint32_t)Q.row_stride();
    ap.ldk = (uint32_t)Kv.row_stride();
    ap.ldv = (uint32_t)V.row_stride();
    ap.ldo = (uint32_t)O.row_stride();
    ap.batch = (uint32_t)B;
    ap.heads = (uint32_t)H;
    ap.q_head_stride = bhsd ? M * ap.ldq : dk;
    ap.q_batch_stride = bhsd ? H * M * ap.ldq : M * ap.ldq;
    ap.k_head_stride = bhsd ? N * ap.ldk : dk;
    ap.k_batch_stride = bhsd ? H * N * ap.ldk : N * ap.ldk;
    ap.v_head_stride = bhsd ? N * ap.ldv : dv;
    ap.v_batch_stride = bhsd ? H * N * ap.ldv : N * ap.ldv;
    ap.o_head_stride = bhsd ? M * ap.ldo : dv;
    ap.o_batch_stride = bhsd ? H * M * ap.ldo : M * ap.ldo;
    // scale=auto: 1/sqrt(head dim), the usual choice the graph cannot state
    ap.scale = attr(op, "scale", "") == "auto" ? (float)(1.0 / std::sqrt((double)dk)) : (float)num("scale", 0.0);
    ap.causal = (uint32_t)num("causal", 0);
    ap.dtype = Q.dtype;
    if (!grad) {
      // A second output receives the per-query log-sum-exp ([batch, heads, seq]).
      float *lse = op.outs.size() > 1 ? f32(op.outs[1]) : nullptr;
      if (lse && val(op.outs[1]).elems() != B * H * M) return bad("lse needs batch*heads*seq elements");
      s = BWPP_PLAN_CALL(lse ? bwpp_hip_dispatch_attention_lse(h, ptr(op.ins[0]), ptr(op.ins[1]), ptr(op.ins[2]), ptr(op.outs[0]),
                                                lse, ap)
              : bwpp_hip_dispatch_attention(h, ptr(op.ins[0]), ptr(op.ins[1]), ptr(op.ins[2]), ptr(op.outs[0]), ap));
    } else {
      s = BWPP_PLAN_CALL(bwpp_hip_attention_grad_planned(h, ptr(op.ins[0]), ptr(op.ins[1]), ptr(op.ins[2]), ptr(op.ins[3]),
                                          ptr(op.ins[4]), f32(op.ins[5]), ptr(op.outs[0]), ptr(op.outs[1]),
                                          ptr(op.outs[2]), ap));
    }
  } else {
    return bad("unknown op");
  }
  if (s != BWPP_HIP_OK) return perr(&p, s, "line %d (%s): %s", op.line, k.c_str(), bwpp_hip_last_error(h));
  return BWPP_HIP_OK;
}

}  // namespace

extern "C" BwppHipStatus bwpp_hip_plan_run(BwppHipPlan *p) {
  if (!p) return BWPP_HIP_ERR_INVALID_ARG;
  if (!p->allocated) return perr(p, BWPP_HIP_ERR_INVALID_ARG, "plan not allocated");
  for (const Value &v : p->values)
    if ((v.kind == Kind::kInput || v.kind == Kind::kParam) && !v.ptr && v.last_use >= 0)
      return perr(p, BWPP_HIP_ERR_INVALID_ARG, "'%s' is not bound", v.name.c_str());
  for (const Op &op : p->ops) {
    BwppHipStatus s = run_op(*p, op);
    if (s != BWPP_HIP_OK) return s;
  }
  return BWPP_HIP_OK;
}

// Memory-plan report in the reference's dump layout (mem_plan.c:176-193:
// "buffers=N values=M", one line per buffer, "vI -> bufferJ"), with the
// byte size and arena offset of each buffer and the arena total appended.
extern "C" size_t bwpp_hip_plan_report(const BwppHipPlan *p, char *buf, size_t cap) {
  if (!p) return 0;
  std::string r;
  char line[512];
  snprintf(line, sizeof line, "buffers=%zu values=%zu\n", p->buffers.size(), p->values.size());
  r += line;
  for (size_t i = 0; i < p->buffers.size(); ++i) {
    const Buffer &b = p->buffers[i];
    std::string shape = "[";
    for (size_t d = 0; d < b.dim_text.size(); ++d) shape += (d ? "," : "") + b.dim_text[d];
    shape += "]";
    snprintf(line, sizeof line, "buffer%zu %s %s row_major bytes=%llu offset=%zu\n", i, dtype_name(b.dtype),
             shape.c_str(), (unsigned long long)b.bytes, b.offset);
    r += line;
  }
  for (size_t i = 0; i < p->values.size(); ++i) {
    const Value &v = p->values[i];
    if (v.buffer < 0) continue;
    snprintf(line, sizeof line, "v%zu -> buffer%d  # %s\n", i, v.buffer, v.name.c_str());
    r += line;
  }
  snprintf(line, sizeof line, "arena_bytes=%zu\n", p->arena_bytes);
  r += line;
  if (buf && cap) {
    const size_t n = r.size() < cap - 1 ? r.size() : cap - 1;
    memcpy(buf, r.data(), n);
    buf[n] = '\0';
  }
  return r.size() + 1;
}
