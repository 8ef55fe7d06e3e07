// Parser for the `nsc --mlir` instruction text (mlir_compiler.cpp:949-1025)
// into a Plan.  The per-op conventions it resolves follow the reference's CPU
// emitter, which is the numeric oracle:
//   weight blob = TENSOR_ALLOC order            codegen.cpp:2442-2444
//   runtime input / labels detection            codegen.cpp:1191-1200, 2693-2706
//   in_cols / out_cols                          codegen.cpp:2295-2320
//   LayerNorm row width (forward / train)       codegen.cpp:2021, 2721-2751
//   activation kind of an ACTIVATION_GRAD       mlir_compiler.cpp:350-359
#include "plan.h"

#include <cctype>
#include <cmath>
#include <cstdlib>
#include <sstream>

namespace nship {
namespace {

std::string trim(const std::string& s) {
  size_t a = 0, b = s.size();
  while (a < b && std::isspace((unsigned char)s[a])) a++;
  while (b > a && std::isspace((unsigned char)s[b - 1])) b--;
  return s.substr(a, b - a);
}

bool starts(const std::string& s, const char* p) { return s.rfind(p, 0) == 0; }

int act_code(const std::string& kind) {
  if (kind == "identity") return 0;
  if (kind == "relu") return 1;
  if (kind == "leaky_relu") return 2;
  if (kind == "sigmoid") return 3;
  if (kind == "tanh") return 4;
  if (kind == "swish" || kind == "silu") return 5;
  if (kind == "gelu") return 6;
  return -1;
}

// key=NUMBER inside a trailing comment, or -1.
int64_t comment_int(const std::string& c, const std::string& key) {
  size_t p = 0;
  while ((p = c.find(key + "=", p)) != std::string::npos) {
    if (p == 0 || !std::isalnum((unsigned char)c[p - 1])) {
      const char* s = c.c_str() + p + key.size() + 1;
      char* e = nullptr;
      long long v = std::strtoll(s, &e, 10);
      if (e != s) return v;
    }
    p += key.size();
  }
  return -1;
}

// VALUE of a key=VALUE token (whitespace-delimited) in a comment, or "".
std::string comment_str(const std::string& c, const std::string& key) {
  size_t p = 0;
  while ((p = c.find(key + "=", p)) != std::string::npos) {
    if (p == 0 || std::isspace((unsigned char)c[p - 1])) {
      size_t e = p + key.size() + 1;
      size_t f = e;
      while (f < c.size() && !std::isspace((unsigned char)c[f])) f++;
      return c.substr(e, f - e);
    }
    p += key.size();
  }
  return "";
}

bool is_fusible(Op op) {  // fusion.cpp:23-40
  return op == Op::Act || op == Op::Softmax || op == Op::LayerNorm || op == Op::Binop;
}

struct Raw {
  std::string op, comment;
  std::vector<std::string> ids;
  std::vector<int64_t> dims;  // -1 = symbolic
  bool has_type = false;
};

bool parse_line(const std::string& line, Raw* r, std::string* err) {
  std::string head = line, comment;
  const size_t c = line.find("//");
  if (c != std::string::npos) {
    head = line.substr(0, c);
    comment = trim(line.substr(c + 2));
  }
  std::string type;
  const size_t colon = head.find(':');
  if (colon != std::string::npos) {
    type = trim(head.substr(colon + 1));
    head = head.substr(0, colon);
  }
  std::istringstream is(head);
  is >> r->op;
  std::string tok;
  while (is >> tok) {
    if (tok[0] != '%') {
      *err = "unexpected token '" + tok + "' in: " + line;
      return false;
    }
    r->ids.push_back(tok.substr(1));
  }
  r->comment = comment;
  if (!type.empty()) {
    const size_t lb = type.find('['), rb = type.find(']');
    if (!starts(type, "Tensor") || lb == std::string::npos || rb == std::string::npos || rb < lb) {
      *err = "bad tensor type in: " + line;
      return false;
    }
    r->has_type = true;
    std::stringstream ds(type.substr(lb + 1, rb - lb - 1));
    std::string d;
    while (std::getline(ds, d, ',')) {
      d = trim(d);
      char* e = nullptr;
      long long v = std::strtoll(d.c_str(), &e, 10);
      r->dims.push_back((!d.empty() && *e == '\0') ? (int64_t)v : -1);
    }
  }
  return true;
}

// `// ns.lr_schedule <kind> warmup=W total=T min=F`; false on a malformed line.
bool parse_lr_schedule(const std::string& line, LrSchedule* s) {
  std::istringstream is(line.substr(line.find("ns.lr_schedule") + 14));
  std::string kind, tok;
  is >> kind;
  if (kind == "constant") s->kind = 0;
  else if (kind == "cosine_warmup") s->kind = 1;
  else return false;
  while (is >> tok) {
    const size_t eq = tok.find('=');
    if (eq == std::string::npos) return false;
    const std::string k = tok.substr(0, eq), v = tok.substr(eq + 1);
    char* e = nullptr;
    if (k == "warmup") s->warmup = std::strtoll(v.c_str(), &e, 10);
    else if (k == "total") s->total = std::strtoll(v.c_str(), &e, 10);
    else if (k == "min") s->min_factor = std::strtof(v.c_str(), &e);
    else return false;
    if (v.empty() || *e != '\0') return false;
  }
  return true;
}

}  // namespace

float lr_scale(const LrSchedule& s, int64_t step) {
  if (s.kind == 0) return 1.0f;
  if (step < s.warmup) return s.warmup > 0 ? (float)step / (float)s.warmup : 1.0f;
  const int64_t end = s.total > s.warmup ? s.total : s.warmup + 1;
  const int64_t st = step >= end ? end : step;
  const float t = (float)(st - s.warmup) / (float)(end - s.warmup);
  return s.min_factor + 0.5f * (1.0f - s.min_factor) * (1.0f + cosf(3.14159265f * t));
}

Plan* parse_plan(const char* text, std::string* err) {
  if (!text) {
    *err = "null IR text";
    return nullptr;
  }
  Plan* P = new Plan();
  auto fail = [&](const std::string& m) -> Plan* {
    *err = m;
    delete P;
    return nullptr;
  };
  auto vid = [&](const std::string& name) -> int {
    auto it = P->index.find(name);
    if (it != P->index.end()) return it->second;
    const int id = (int)P->vals.size();
    P->vals.push_back(Value{name});
    P->index[name] = id;
    return id;
  };

  struct RawFunc {
    std::string name;
    std::vector<Raw> ins;
    std::string ret;
    bool train = false;
  };
  std::vector<RawFunc> funcs;
  RawFunc* cur = nullptr;
  std::istringstream in(text);
  std::string line;
  while (std::getline(in, line)) {
    line = trim(line);
    if (starts(line, "// ns.lr_schedule")) {
      if (!parse_lr_schedule(line, &P->lr)) return fail("bad lr schedule line: " + line);
      continue;
    }
    if (line.empty() || starts(line, "//")) continue;
    if (starts(line, "ns.func @")) {
      funcs.push_back(RawFunc());
      cur = &funcs.back();
      std::istringstream ls(line.substr(9));
      ls >> cur->name;
      continue;
    }
    if (line == "}") {
      cur = nullptr;
      continue;
    }
    if (!cur) return fail("instruction outside a function: " + line);
    if (starts(line, "ns.return")) {
      const size_t p = line.find('%');
      if (p == std::string::npos) return fail("bad return: " + line);
      cur->ret = trim(line.substr(p + 1));
      continue;
    }
    Raw r;
    if (!parse_line(line, &r, err)) {
      delete P;
      return nullptr;
    }
    if (r.op == "ns.grad") cur->train = true;
    cur->ins.push_back(r);
  }
  const RawFunc* rf = nullptr;
  const RawFunc* rt = nullptr;
  for (auto& f : funcs) {
    if (!f.train && !rf) rf = &f;
    if (f.train && !rt) rt = &f;
  }
  if (!rf) return fail("IR has no forward function");

  // Weights in TENSOR_ALLOC order of the forward function.
  for (auto& r : rf->ins) {
    if (r.op != "ns.tensor.alloc") continue;
    if (r.ids.size() != 1 || r.dims.empty()) return fail("bad alloc");
    const int id = vid(r.ids[0]);
    Value& v = P->vals[id];
    v.weight = true;
    v.rows = r.dims[0];
    v.cols = r.dims.size() > 1 ? r.dims[1] : 1;
    if (v.rows <= 0 || v.cols <= 0) return fail("weight '" + v.name + "' has a dynamic shape");
    v.offset = P->total;
    P->total += (size_t)(v.rows * v.cols);
    P->weights.push_back(id);
  }

  auto build = [&](const RawFunc& f, Func* F) -> bool {
    F->name = f.name;
    F->train = f.train;
    std::vector<int64_t> rt(0);
    auto rtc = [&](int id) -> int64_t& {
      if ((int)rt.size() <= id) rt.resize(id + 1, -1);
      return rt[id];
    };
    for (auto& r : f.ins) {
      Instr I;
      const std::string& o = r.op;
      size_t nres = 1;
      if (o == "ns.tensor.alloc") { I.op = Op::Alloc; }
      else if (o == "ns.grad" || o == "ns.forward") { I.op = Op::Marker; nres = 0; }
      else if (o == "ns.matmul") I.op = Op::Matmul;
      else if (o == "ns.activation.softmax") I.op = Op::Softmax;
      else if (o == "ns.subview_binop") {
        I.op = Op::Binop;
        const std::string b = comment_str(r.comment, "op");
        I.binop = b == "-" ? 1 : b == "*" ? 2 : b == "/" ? 3 : 0;  // codegen.cpp:2010-2013
      }
      else if (o == "ns.constant") {
        I.op = Op::Constant;
        std::string v = comment_str(r.comment, "value");
        if (v.empty()) {  // "constant <literal>"
          const size_t sp = r.comment.rfind(' ');
          v = sp == std::string::npos ? r.comment : r.comment.substr(sp + 1);
        }
        char* e = nullptr;
        I.value = (float)std::strtod(v.c_str(), &e);
        if (e == v.c_str()) { *err = "bad constant: " + r.comment; return false; }
      }
      else if (o == "ns.transpose") I.op = Op::Transpose;
      else if (o == "ns.reshape") I.op = Op::Reshape;
      else if (o == "ns.concat" || o == "ns.slice" || o == "ns.index" || o == "ns.scatter") {
        I.op = o == "ns.concat" ? Op::Concat : o == "ns.slice" ? Op::Slice : o == "ns.index" ? Op::Index : Op::Scatter;
        const std::string ax = comment_str(r.comment, "axis");
        if (ax.empty()) { *err = o + " without its axis= attribute (use the attribute-preserving IR printer)"; return false; }
        I.axis = std::atoi(ax.c_str());
        if (I.op == Op::Concat) I.axis = ax == "0" ? 0 : 1;  // codegen.cpp:2105
        if (I.op == Op::Slice) {
          I.start = comment_int(r.comment, "start");
          I.stop = comment_int(r.comment, "stop");
          if (I.start < 0 || I.stop < I.start) { *err = "bad slice range: " + r.comment; return false; }
        }
        if (I.op == Op::Index || I.op == Op::Scatter) {
          std::stringstream ls(comment_str(r.comment, "idx"));
          std::string t;
          while (std::getline(ls, t, ',')) {
            if (t.empty()) continue;
            char* e = nullptr;
            const long long v = std::strtoll(t.c_str(), &e, 10);
            if (*e != '\0') { *err = "bad index list: " + r.comment; return false; }
            I.idx.push_back(v);
          }
        }
      }
      else if (starts(o, "ns.activation.")) {
        I.op = Op::Act;
        I.act = act_code(o.substr(14));
        if (I.act < 0) { *err = "unsupported activation: " + o; return false; }
      }
      else if (o == "ns.dropout") {
        I.op = Op::Dropout;
        const std::string v = comment_str(r.comment, "rate");
        I.rate = v.empty() ? 0.0 : std::strtod(v.c_str(), nullptr);
      }
      else if (o == "ns.layernorm") I.op = Op::LayerNorm;
      else if (o == "ns.layer.embedding") I.op = Op::Embedding;
      else if (o == "ns.layer.attention") I.op = Op::Attention;
      else if (o == "ns.layer.moe") I.op = Op::Moe;
      else if (o == "ns.cross_entropy") I.op = Op::CrossEntropy;
      else if (o == "ns.grad.loss") I.op = Op::LossGrad;
      else if (o == "ns.grad.matmul.a") I.op = Op::MatmulGradA;
      else if (o == "ns.grad.matmul.w") I.op = Op::MatmulGradW;
      else if (o == "ns.grad.activation") {
        // a dropout's gradient multiplies by the saved mask
        // (mlir_compiler.cpp:362-375: operand 1 is the dropout's result)
        I.op = Op::ActGrad;
        I.dropout = r.comment.find("dropout_mask") != std::string::npos;
      }
      else if (o == "ns.grad.layernorm") I.op = Op::LayerNormGrad;
      else if (o == "ns.grad.embedding.w") I.op = Op::EmbeddingGradW;
      else if (o == "ns.grad.attention.x") I.op = Op::AttnGradX;
      else if (o == "ns.grad.attention.wq") I.op = Op::AttnGradWq;
      else if (o == "ns.grad.attention.wk") I.op = Op::AttnGradWk;
      else if (o == "ns.grad.attention.wv") I.op = Op::AttnGradWv;
      else if (o == "ns.grad.attention.wo") I.op = Op::AttnGradWo;
      else if (o == "ns.grad.moe.x") I.op = Op::MoeGradX;
      else if (o == "ns.grad.moe.wg") I.op = Op::MoeGradWg;
      else if (o == "ns.grad.moe.we1") I.op = Op::MoeGradWe1;
      else if (o == "ns.grad.moe.we2") I.op = Op::MoeGradWe2;
      else if (o == "ns.opt.step") { I.op = Op::OptStep; nres = 0; }
      else { *err = "unsupported instruction: " + o; return false; }
      if (I.op == Op::Alloc) {
        auto it = P->index.find(r.ids[0]);
        if (it == P->index.end() || !P->vals[it->second].weight) {
          *err = "train function allocates a weight the forward does not: " + r.ids[0];
          return false;
        }
        continue;
      }
      if (r.ids.size() < nres) { *err = "missing result id: " + o; return false; }
      if (nres) I.res = vid(r.ids[0]);
      for (size_t k = nres; k < r.ids.size(); k++) I.in.push_back(vid(r.ids[k]));
      static const std::map<Op, size_t> arity = {
          {Op::Matmul, 2}, {Op::Act, 1}, {Op::Dropout, 1}, {Op::LayerNorm, 1}, {Op::Embedding, 2},
          {Op::Attention, 5}, {Op::Moe, 4}, {Op::CrossEntropy, 2}, {Op::LossGrad, 2},
          {Op::MatmulGradA, 2}, {Op::MatmulGradW, 3}, {Op::ActGrad, 2}, {Op::LayerNormGrad, 2},
          {Op::EmbeddingGradW, 3}, {Op::AttnGradX, 6}, {Op::AttnGradWq, 6}, {Op::AttnGradWk, 6},
          {Op::AttnGradWv, 6}, {Op::AttnGradWo, 6}, {Op::MoeGradX, 5}, {Op::MoeGradWg, 5},
          {Op::MoeGradWe1, 5}, {Op::MoeGradWe2, 5}, {Op::Binop, 2}, {Op::Softmax, 1}, {Op::Transpose, 1},
          {Op::Concat, 2}, {Op::Reshape, 1}, {Op::Slice, 1}, {Op::Index, 1}, {Op::Scatter, 2}};
      auto ar = arity.find(I.op);
      if (ar != arity.end() && I.in.size() < ar->second) { *err = "too few operands: " + o; return false; }
      if (I.op == Op::OptStep && I.in.size() % 2) { *err = "odd ns.opt.step operand list"; return false; }
      if (I.op == Op::OptStep) {
        const std::string opt = comment_str(r.comment, "optimizer");
        if (!opt.empty() && opt != "adamw") { *err = "unknown optimizer= " + opt; return false; }
        I.adamw_only = opt == "adamw";
      }
      if (I.res >= 0 && r.has_type && r.dims.size() > 1) rtc(I.res) = r.dims[1];
      if (I.res >= 0) {
        if ((int)F->srows.size() <= I.res) { F->srows.resize(I.res + 1, -1); F->scols.resize(I.res + 1, -1); }
        F->srows[I.res] = r.has_type && !r.dims.empty() ? r.dims[0] : -1;
        F->scols[I.res] = r.has_type && r.dims.size() > 1 ? r.dims[1] : -1;
      }
      I.rt_cols = I.res >= 0 ? rtc(I.res) : -1;
      if (I.op == Op::Attention) {
        const int64_t h = comment_int(r.comment, "heads");
        I.heads = h > 0 ? (int)h : 1;
      }
      if (I.op == Op::Moe) {
        // MoE(initial_experts: K0) lives only in the instruction's ints
        // attribute (mlir_compiler.cpp:896), which the plain `nsc --mlir`
        // printer drops (:899-902); without it the liveness mask is unknown,
        // so the plan is refused rather than assuming every expert live.
        // K0 <= 0 or > E means all E (mlir_compiler.cpp:194-195).
        const int64_t k0 = comment_int(r.comment, "initial");
        if (k0 < 0 && r.comment.find("initial=") == std::string::npos) {
          *err = "ns.layer.moe needs initial=K0 in its comment (the plain nsc --mlir text omits "
                 "MoE initial_experts; print the IR with oracle/irdump): " + o;
          return false;
        }
        MoeInfo& m = P->moe;
        const Value& g = P->vals[I.in[1]];
        const Value& e1 = P->vals[I.in[2]];
        if (!g.weight || !e1.weight || !P->vals[I.in[3]].weight) { *err = "moe operands must be weights"; return false; }
        if (m.present && m.g != I.in[1]) { *err = "only one MoE layer per model is supported"; return false; }
        m.present = true;
        m.D = g.rows;
        m.E = g.cols;
        m.H = e1.cols / m.D;
        m.K0 = (k0 > 0 && k0 <= m.E) ? k0 : m.E;
        m.g = I.in[1];
        m.e1 = I.in[2];
        m.e2 = I.in[3];
        if (e1.rows != m.E || e1.cols != m.D * m.H || P->vals[m.e2].cols != m.H * m.D) {
          *err = "inconsistent MoE weight shapes";
          return false;
        }
      }
      F->ins.push_back(I);
    }
    F->ret = f.ret.empty() ? -1 : vid(f.ret);
    // attention heads and activation kinds for the grads
    for (auto& I : F->ins) {
      if (I.op >= Op::AttnGradX && I.op <= Op::AttnGradWo) {
        bool found = false;
        for (auto& J : F->ins)
          if (J.op == Op::Attention && J.in[1] == I.in[2]) { I.heads = J.heads; found = true; }
        if (!found) { *err = "attention grad without its forward"; return false; }
      }
      if (I.op == Op::ActGrad && I.dropout) {
        bool found = false;
        for (auto& J : F->ins)
          if (J.op == Op::Dropout && J.res == I.in[1]) { I.rate = J.rate; found = true; }
        if (!found) { *err = "dropout grad without its forward"; return false; }
      } else if (I.op == Op::ActGrad) {
        bool found = false;
        for (auto& J : F->ins) {
          if (J.op == Op::Act && J.in[0] == I.in[1]) { I.act = J.act; found = true; }
          // softmax's gradient is emitted as ACTIVATION_GRAD "softmax", whose
          // derivative code is 0, i.e. 1 (mlir_compiler.cpp:348-360,
          // codegen.cpp:3074-3081, 1305-1315)
          if (J.op == Op::Softmax && J.in[0] == I.in[1]) { I.act = 0; found = true; }
        }
        if (!found) { *err = "activation grad without its forward"; return false; }
      }
    }
    // runtime input / labels
    auto is_w = [&](int id) { return P->vals[id].weight; };
    for (auto& I : F->ins) {
      int cand = -1;
      if (I.op == Op::Embedding) cand = I.in[1];
      else if (I.op == Op::Matmul) cand = I.in[0];
      else if (!F->train && (I.op == Op::Attention || I.op == Op::LayerNorm || I.op == Op::Moe ||
                             I.op == Op::Dropout || I.op == Op::Act || I.op == Op::Softmax ||
                             I.op == Op::Transpose || I.op == Op::Concat || I.op == Op::Reshape ||
                             I.op == Op::Slice || I.op == Op::Index || I.op == Op::Scatter))
        cand = I.in[0];  // codegen.cpp:44-61
      if (cand >= 0 && !is_w(cand)) { F->x = cand; break; }
    }
    for (auto& I : F->ins)
      if (I.op == Op::CrossEntropy) F->y = I.in[1];
    if (F->x < 0) { *err = "cannot find the runtime input of " + f.name; return false; }
    // static shape table: weights, result types, and the input's width
    // (first GEMM's K, else 1; codegen.cpp:1209-1224)
    F->srows.resize(P->vals.size() + 1, -1);
    F->scols.resize(P->vals.size() + 1, -1);
    for (size_t id = 0; id < P->vals.size(); id++)
      if (P->vals[id].weight) { F->srows[id] = P->vals[id].rows; F->scols[id] = P->vals[id].cols; }
    {
      int64_t in_w = 1;
      for (auto& I : F->ins) {
        if (I.op == Op::Matmul) { in_w = F->srows[I.in[1]]; break; }
        if (I.op == Op::Embedding) break;
      }
      F->scols[F->x] = in_w;
    }
    // GEMM shapes from the B operand's static shape (a weight or a typed value)
    for (auto& I : F->ins) {
      if (I.op != Op::Matmul) continue;
      I.k = F->srows[I.in[1]];
      I.n = F->scols[I.in[1]];
      if (I.k <= 0 || I.n <= 0) {
        *err = "matmul operand '" + P->vals[I.in[1]].name + "' has no static shape";
        return false;
      }
    }
    // The reference's fusion pass (fusion.cpp:52-175): a GEMM whose result has
    // one use absorbs the run of fusible ops that each consume the previous
    // one's result and are used at most once (the last one any number of times
    // when it ends the run... it must be used <= 1 unless it is last).
    {
      std::vector<int> uses(P->vals.size() + 1, 0);
      for (auto& I : F->ins)
        for (int v : I.in) uses[v]++;
      for (size_t i = 0; i < F->ins.size(); i++) {
        const Instr& lead = F->ins[i];
        if (lead.op != Op::Matmul || uses[lead.res] != 1) continue;
        size_t end = i + 1;
        int consumed = lead.res;
        while (end < F->ins.size()) {
          const Instr& c = F->ins[end];
          if (!is_fusible(c.op) || c.in.empty() || c.in[0] != consumed) break;
          const bool last = end + 1 >= F->ins.size() || !is_fusible(F->ins[end + 1].op) ||
                            F->ins[end + 1].in.empty() || F->ins[end + 1].in[0] != c.res;
          if (uses[c.res] > 1 || (!last && uses[c.res] == 0)) break;
          consumed = c.res;
          end++;
        }
        if (end == i + 1) continue;
        if (F->train) {
          *err = "fused epilogue groups in train() are not supported (the reference's train core skips them)";
          return false;
        }
        for (size_t j = i + 1; j < end; j++) {
          F->ins[j].in_group = true;
          F->ins[j].group_n = lead.n;
        }
        i = end - 1;
      }
    }
    if (F->train) {
      for (auto& I : F->ins)
        if (I.op == Op::Binop || I.op == Op::Constant || (I.op >= Op::Transpose && I.op <= Op::Scatter)) {
          *err = "binop / data-movement instructions in train() are not supported (the reference's train core "
                 "skips them)";
          return false;
        }
    }
    // column widths: static result types first, then the reference's
    // forward propagation (codegen.cpp:2721-2741).
    F->width.assign(P->vals.size() + 1, -1);
    for (size_t id = 0; id < P->vals.size(); id++) {
      if (P->vals[id].weight) F->width[id] = P->vals[id].cols;
      else if (id < rt.size() && rt[id] > 0) F->width[id] = rt[id];
    }
    for (auto& I : F->ins) {
      if (I.res < 0) continue;
      if (I.op == Op::Matmul) F->width[I.res] = I.n;
      else if (I.op == Op::Constant) F->width[I.res] = 1;
      else if (!I.in.empty() && F->width[I.res] <= 0 && F->width[I.in[0]] > 0)
        F->width[I.res] = F->width[I.in[0]];
    }
    return true;
  };

  if (!build(*rf, &P->fwd)) { delete P; return nullptr; }
  if (rt) {
    if (!build(*rt, &P->trn)) { delete P; return nullptr; }
    P->has_train = true;
    if (P->trn.y < 0) return fail("train function has no cross_entropy");
  }

  // in_cols / out_cols (codegen.cpp:2295-2320)
  {
    const Func& F = P->fwd;
    int64_t in_c = -1, out_c = -1;
    auto rtcols = [&](int id) -> int64_t {
      for (auto& I : F.ins) if (I.res == id) return I.rt_cols;
      return -1;
    };
    for (auto& I : F.ins)
      if (I.res >= 0 && I.res == F.ret) out_c = rtcols(I.res);
    for (auto& I : F.ins) {
      if (I.in_group) continue;  // absorbed by a GEMM group: not in the emitted list
      if (I.op == Op::Matmul) {
        if (in_c < 0) in_c = I.k;
        out_c = I.n;
      }
      if (I.op == Op::Embedding && in_c < 0) in_c = 1;
      if ((I.op == Op::Attention || I.op == Op::LayerNorm || I.op == Op::Moe || I.op == Op::Softmax ||
           I.op == Op::Concat || I.op == Op::Slice || I.op == Op::Index || I.op == Op::Scatter ||
           I.op == Op::Transpose || I.op == Op::Reshape) &&
          I.res >= 0) {
        const int64_t c = rtcols(I.res);
        if (c > 0) out_c = c;
      }
    }
    P->in_cols = in_c > 0 ? in_c : 1;
    P->out_cols = out_c > 0 ? out_c : 1;
    // the raw input's width (codegen.cpp:1203-1216)
    if (P->fwd.x >= 0) P->fwd.width[P->fwd.x] = P->in_cols;
  }

  // Forward peephole: Matmul whose only consumer is the next Act gets that
  // activation as its epilogue (the fusion pass, fusion.cpp:112-157).
  {
    Func& F = P->fwd;
    for (size_t i = 0; i + 1 < F.ins.size(); i++) {
      Instr& mm = F.ins[i];
      Instr& ac = F.ins[i + 1];
      if (mm.op != Op::Matmul || ac.op != Op::Act || ac.in[0] != mm.res || mm.res == F.ret) continue;
      int uses = 0;
      for (auto& J : F.ins)
        for (int v : J.in) uses += v == mm.res;
      if (uses != 1) continue;
      mm.act = ac.act;
      mm.res = ac.res;
      ac.fused_away = true;
    }
  }

  for (int id : P->weights) P->wnames.push_back(P->vals[id].name);
  for (size_t i = 0; i < P->weights.size(); i++) {
    const Value& v = P->vals[P->weights[i]];
    P->desc.push_back(ns_weight_desc{P->wnames[i].c_str(), v.offset, (size_t)(v.rows * v.cols)});
  }
  P->layout.num_weights = P->desc.size();
  P->layout.desc = P->desc.empty() ? nullptr : P->desc.data();
  return P;
}

}  // namespace nship
