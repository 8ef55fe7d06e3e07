// libnship runtime: plans, models, the instruction executor and the C-ABI
// (include/nship.h).  Replaces the per-network driver the reference emits
// (CPU: /root/reference/src/codegen/codegen.cpp:2290-2654, CUDA: :916-1127)
// with one runtime that walks the parsed instruction list and launches the
// hand-written gfx950 kernels on the model's private stream.
//
// Memory: the weight blob lives in HBM for the model's lifetime (the CPU
// reference re-copies it on every call, codegen.cpp:2268-2273); activations
// live in a grow-only per-value arena sized on the first call of a given
// batch; the host blob copy is refreshed lazily after training.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <random>
#include <string>
#include <vector>

#include "common.h"
#include "hostcopy.h"
#include "kernels.h"
#include "nship.h"
#include "plan.h"

namespace nship {

static thread_local std::string g_err;
void set_error(const std::string& msg) { g_err = msg; }

namespace {

struct Buf {
  float* p = nullptr;
  size_t cap = 0;  // floats
};

struct ProfEntry {
  const char* name;
  hipEvent_t a, b;
};

}  // namespace
}  // namespace nship

using namespace nship;

struct nsh_plan {
  std::unique_ptr<Plan> p;
  ns_model* fwd = nullptr;  // the model behind nsh_forward, made on its first call
};

struct ns_model {
  const Plan* plan = nullptr;
  hipStream_t stream = nullptr;
  float* d_w = nullptr;
  std::vector<float> h_w;
  bool host_stale = false;  // device blob newer than h_w
  bool device_stale = false;  // h_w newer than the device blob (a failed upload)
  bool mask_stale = false;    // moe_active newer than d_active (a failed mask upload)
  std::vector<uint8_t> moe_active;
  size_t moe_count = 0;
  uint8_t* d_active = nullptr;
  std::mt19937 rng{0x9E3779B9u};  // codegen.cpp:2421
  std::map<int, std::vector<uint8_t>> drop_keep;  // host staging of each dropout's keep flags
  int64_t lr_step = 0;
  int64_t moe_last_m = 0;         // tokens routed by the last MoE forward
  // the expert weight gradients' per-expert nonzero flags and the buffers
  // they describe (MoeBwdWork::dirty)
  const void* moe_dirty_for[3] = {nullptr, nullptr, nullptr};
  struct Adam {
    float* m = nullptr;
    float* v = nullptr;
    int64_t t = 0;
  };
  std::map<int, Adam> adam;       // AdamW state per weight value id
  std::vector<MuonMat> muon_host; // descriptors of the last optimizer step
  std::vector<float*> last_ptr;   // value buffers of the last call (read-back)
  std::vector<size_t> last_numel;
  std::vector<Buf> arena;         // per value id
  std::map<std::string, Buf> scratch;
  std::map<int, int64_t*> dev_idx;  // Index / Scatter index lists on the device, by result id
  nship::HostStage stage;           // pinned staging of the host-pointer entry points' copies
  // Host labels of a host-pointer train call, uploaded when the loss first
  // needs them (on copy_stream, so the upload overlaps the forward pass)
  const float* labels_host = nullptr;
  float* labels_dev = nullptr;
  size_t labels_bytes = 0;
  hipStream_t copy_stream = nullptr;
  hipEvent_t labels_ev = nullptr;
  hipEvent_t before_ev = nullptr;   // the model's stream before this call's kernels
  // Muon's sliced-path stream (created when a step has both long and short
  // Muon matrices), forked from and joined back to `stream` inside a step
  nship::MgsSide muon_side;
  // profiling
  bool prof = false;
  std::vector<std::string> prof_sel;  // regions to time (empty: every region)
  std::vector<ProfEntry> pending;
  std::vector<hipEvent_t> event_pool;
  std::map<std::string, std::pair<long, double>> prof_acc;
};

namespace nship {
namespace {

int ensure(Buf& b, size_t n) {
  if (n <= b.cap && b.p) return 0;  // (an empty request still gets a buffer)
  if (b.p) NSH_CHECK(hipFree(b.p));
  b.p = nullptr;
  b.cap = 0;
  NSH_CHECK(hipMalloc(&b.p, (n ? n : 1) * sizeof(float)));
  b.cap = n;
  return 0;
}

hipEvent_t take_event(ns_model* m) {
  if (!m->event_pool.empty()) {
    hipEvent_t e = m->event_pool.back();
    m->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Records an event pair around one launch when profiling is on.
struct Prof {
  ns_model* m;
  const char* name;
  hipEvent_t a = nullptr;
  Prof(ns_model* mm, const char* n) : m(mm), name(n) {
    if (m->prof && selected() && (a = take_event(m))) hipEventRecord(a, m->stream);
  }
  bool selected() const {
    if (m->prof_sel.empty()) return true;
    for (const std::string& r : m->prof_sel)
      if (r == name) return true;
    return false;
  }
  ~Prof() {
    if (!a) return;
    hipEvent_t b = take_event(m);
    if (!b) return;
    hipEventRecord(b, m->stream);
    m->pending.push_back(ProfEntry{name, a, b});
  }
};

void collect_profile(ns_model* m) {
  for (auto& e : m->pending) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, e.a, e.b) == hipSuccess) {
      auto& acc = m->prof_acc[e.name];
      acc.first += 1;
      acc.second += ms;
    }
    m->event_pool.push_back(e.a);
    m->event_pool.push_back(e.b);
  }
  m->pending.clear();
}

int sync(ns_model* m) {
  NSH_CHECK(hipStreamSynchronize(m->stream));
  if (m->prof) collect_profile(m);
  return 0;
}

// Elementwise activation (forward ops that were not fused into a GEMM).
__global__ void act_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n, int code) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = act_apply(x[i], code);
}

// Per-call shapes and device pointers of every value of a function.
struct AttnSaved {
  float* qkv = nullptr;  // [3][BS][D]
  float* ctx = nullptr;  // [BS][D] per-head outputs before the projection
  float* lse = nullptr;  // [H][BS]
  int64_t BS = 0;
};

struct Frame {
  std::vector<size_t> numel;
  std::vector<float*> ptr;
  std::map<int, AttnSaved> attn;  // keyed by the attention input value id
  bool backward = false;          // train_mode: a backward pass and optimizer step follow
  // sign bits of a relu layer's pre-activation (by its value id) and their
  // pitch, written by the training forward's GEMM for the backward's relu'
  // epilogue (GemmArgs::mask_out / mask_in)
  std::map<int, std::pair<uint16_t*, int64_t>> relu_bits;
  // a value the caller's buffer receives directly (the device-pointer
  // forward's return value), or -1; not when that buffer would overlap the
  // input [direct_in, direct_in + direct_in_n), which the producing
  // instruction may still read
  int direct_id = -1;
  float* direct = nullptr;
  const float* direct_in = nullptr;
  size_t direct_in_n = 0;
  // embedding weight gradients (by value id) and their token counts: at most
  // that many of their rows are nonzero
  std::map<int, int64_t> emb_tokens;
};

float* scratch(ns_model* m, const std::string& key, size_t n) {
  Buf& b = m->scratch[key];
  if (ensure(b, n) != 0) return nullptr;
  return b.p;
}

// GEMMs of the model's plan: split K through a grow-only workspace when the
// output has too few tiles to fill the device (weight gradients).
int rt_gemm_ex(ns_model* m, const GemmArgs& g, bool tA, bool tB, int batch) {
  const int sp = gemm_split_count(g, batch);
  if (sp <= 1) return launch_gemm_ex(g, tA, tB, batch, m->stream);
  float* ws = scratch(m, "splitk", gemm_split_workspace(g, batch, sp));
  if (!ws) return -1;
  return launch_gemm_split(g, tA, tB, batch, sp, ws, m->stream);
}

int rt_gemm(ns_model* m, const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K, int64_t lda,
            int64_t ldb, int64_t ldc, bool tA, bool tB, int act) {
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) {
    set_error("gemm: dimension exceeds int32");
    return -1;
  }
  GemmArgs g;
  g.A = A; g.B = B; g.C = C;
  g.M = (int)M; g.N = (int)N; g.K = (int)K;
  g.lda = lda; g.ldb = ldb; g.ldc = ldc;
  g.act = act;
  return rt_gemm_ex(m, g, tA, tB, 1);
}

// MoE work arrays for M tokens (grow-only scratch).
int moe_work(ns_model* m, int64_t M, MoeWork* w) {
  const MoeInfo& q = m->plan->moe;
  float* lg = scratch(m, "moe_logits", (size_t)(M * q.E));
  float* pr = scratch(m, "moe_prob", (size_t)M);
  float* hid = scratch(m, "moe_hidden", (size_t)(M * q.H));
  int* iw = reinterpret_cast<int*>(scratch(m, "moe_ints", moe_work_ints(M, q.E)));
  if (!lg || !pr || !hid || !iw) return -1;
  const int64_t nblk = ceil_div(M, 256);
  w->logits = lg;
  w->prob = pr;
  w->hidden = hid;
  w->best = iw;
  w->rank = iw + M;
  w->perm = iw + 2 * M;
  w->bcount = iw + 3 * M;
  w->seg = w->bcount + nblk * q.E;
  w->tiles = w->seg + q.E + 1;
  w->ntiles = w->tiles + 2 * (ceil_div(M, 128) + q.E + 1);
  w->pre = nullptr;
  return 0;
}

int bind_weights(ns_model* m, Frame& fr) {
  const Plan& P = *m->plan;
  fr.numel.assign(P.vals.size(), 0);
  fr.ptr.assign(P.vals.size(), nullptr);
  for (int id : P.weights) {
    const Value& v = P.vals[id];
    fr.numel[id] = (size_t)(v.rows * v.cols);
    fr.ptr[id] = m->d_w + v.offset;
  }
  return 0;
}

void keep_frame(ns_model* m, const Frame& fr) {
  m->last_ptr = fr.ptr;
  m->last_numel = fr.numel;
}

float* out_buf(ns_model* m, Frame& fr, int id, size_t n) {
  if (id == fr.direct_id &&
      (fr.direct + n <= fr.direct_in || fr.direct_in + fr.direct_in_n <= fr.direct)) {
    fr.numel[id] = n;
    fr.ptr[id] = fr.direct;
    return fr.direct;
  }
  if (ensure(m->arena[id], n) != 0) return nullptr;
  fr.numel[id] = n;
  fr.ptr[id] = m->arena[id].p;
  return fr.ptr[id];
}

#define NSH_OUT(var, id, n)                          \
  float* var = out_buf(m, fr, (id), (n));            \
  if (!var) return -1

// Forward instructions (shared by inference and the training forward).
// A dropout's rate as the emitted code spells it: clamped to [0, 0.999999]
// and printed with std::to_string into the source (codegen.cpp:2877-2880).
double dropout_rate(double rate) {
  if (rate < 0.0) rate = 0.0;
  if (rate >= 1.0) rate = 0.999999;
  return std::strtod(std::to_string(rate).c_str(), nullptr);
}

float dropout_scale(double r) { return 1.0f / (float)(1.0 - r); }

// Device keep flags (one byte per element) of the dropout whose result is `res`.
uint8_t* drop_mask(ns_model* m, int res, size_t n) {
  float* p = scratch(m, "dropmask" + std::to_string(res), (n + 3) / 4);
  return reinterpret_cast<uint8_t*>(p);
}

int exec_forward_op(ns_model* m, const Func& F, const Instr& I, Frame& fr, bool train) {
  const Plan& P = *m->plan;
  hipStream_t s = m->stream;
  switch (I.op) {
    case Op::Matmul: {
      const int64_t K = I.k, N = I.n;  // B: a weight or a statically shaped value
      const int64_t M = (int64_t)(fr.numel[I.in[0]] / (size_t)K);
      if (fr.numel[I.in[1]] < (size_t)(K * N)) {
        set_error("matmul: operand '" + P.vals[I.in[1]].name + "' is smaller than its static shape");
        return -1;
      }
      NSH_OUT(C, I.res, (size_t)(M * N));
      Prof p(m, I.act ? "gemm_act" : "gemm");
      return rt_gemm(m, fr.ptr[I.in[0]], fr.ptr[I.in[1]], C, M, N, K, K, N, N, false, false, I.act);
    }
    case Op::Act: {
      const size_t n = fr.numel[I.in[0]];
      NSH_OUT(y, I.res, n);
      Prof p(m, "act");
      if (n) {
        hipLaunchKernelGGL(act_kernel, dim3((unsigned)ceil_div((int64_t)n, 256)), dim3(256), 0, s,
                           fr.ptr[I.in[0]], y, (int64_t)n, I.act);
        NSH_LAUNCHED();
      }
      return 0;
    }
    case Op::Embedding: {
      const Value& W = P.vals[I.in[0]];
      const size_t n = fr.numel[I.in[1]];
      NSH_OUT(out, I.res, n * (size_t)W.cols);
      Prof p(m, "embedding");
      return launch_embedding(fr.ptr[I.in[0]], fr.ptr[I.in[1]], out, (int64_t)n, W.rows, W.cols, s);
    }
    case Op::LayerNorm: {
      // row width: the result type's columns, else the input's
      // (codegen.cpp:2021 forward, :2744-2751 train)
      int64_t last = train ? F.width[I.in[0]] : (I.rt_cols > 0 ? I.rt_cols : F.width[I.in[0]]);
      if (I.in_group) last = I.group_n;  // inside a GEMM group: rows of N (codegen.cpp:2066-2067)
      if (last <= 0) last = 1;
      const size_t n = fr.numel[I.in[0]];
      NSH_OUT(y, I.res, n);
      Prof p(m, "layernorm");
      return launch_layernorm(fr.ptr[I.in[0]], y, (int64_t)(n / (size_t)last), last, s);
    }
    case Op::Attention: {
      const Value& Wq = P.vals[I.in[1]];
      const int64_t D = Wq.rows, H = I.heads;
      const int64_t BS = (int64_t)(fr.numel[I.in[0]] / (size_t)D);
      NSH_OUT(out, I.res, (size_t)(BS * D));
      const std::string key = std::to_string(I.res);
      AttnSaved sv;
      sv.BS = BS;
      sv.qkv = scratch(m, "qkv" + key, (size_t)(3 * BS * D));
      sv.ctx = scratch(m, "ctx" + key, (size_t)(BS * D));
      sv.lse = scratch(m, "lse" + key, (size_t)(H * BS));
      if (!sv.qkv || !sv.ctx || !sv.lse) return -1;
      fr.attn[I.in[0]] = sv;
      if (BS == 0) return 0;
      // Q, K, V projections: one batched launch when the three weights are
      // consecutive in the blob (they are for every Attention layer).
      const Value& Wk = P.vals[I.in[2]];
      const Value& Wv = P.vals[I.in[3]];
      const bool packed = Wk.offset == Wq.offset + (size_t)(D * D) && Wv.offset == Wk.offset + (size_t)(D * D);
      {
        Prof p(m, "gemm");
        GemmArgs g;
        g.A = fr.ptr[I.in[0]];
        g.M = (int)BS; g.N = (int)D; g.K = (int)D;
        g.lda = D; g.ldb = D; g.ldc = D;
        if (packed) {
          g.B = fr.ptr[I.in[1]];
          g.C = sv.qkv;
          g.sA = 0; g.sB = D * D; g.sC = BS * D;
          if (rt_gemm_ex(m, g, false, false, 3) != 0) return -1;
        } else {
          for (int j = 0; j < 3; j++) {
            g.B = fr.ptr[I.in[1 + j]];
            g.C = sv.qkv + j * BS * D;
            if (rt_gemm_ex(m, g, false, false, 1) != 0) return -1;
          }
        }
      }
      {
        Prof p(m, "attention_fwd");
        const void* qkv[3] = {sv.qkv, sv.qkv + BS * D, sv.qkv + 2 * BS * D};
        float* pad = nullptr;
        if (!attention_in_place(D, H, D, qkv, 3) && !(pad = scratch(m, "attn_pad", attention_pad_floats(BS, D, H, false))))
          return -1;
        if (launch_attention_fwd(sv.qkv, sv.qkv + BS * D, sv.qkv + 2 * BS * D, sv.ctx, train ? sv.lse : nullptr, BS, D,
                                 H, D, pad, s) != 0)
          return -1;
      }
      Prof p(m, "gemm");
      return rt_gemm(m, sv.ctx, fr.ptr[I.in[4]], out, BS, D, D, D, D, D, false, false, 0);
    }
    case Op::Moe: {
      const MoeInfo& q = P.moe;
      const int64_t M = (int64_t)(fr.numel[I.in[0]] / (size_t)q.D);
      NSH_OUT(out, I.res, (size_t)(M * q.D));
      MoeWork w;
      if (moe_work(m, M, &w) != 0) return -1;
      if (train && !(w.pre = scratch(m, "moe_pre", (size_t)(M * q.H)))) return -1;
      {
        Prof p(m, "moe_route");  // router logits, expert choice, stable dispatch
        if (launch_moe_route(fr.ptr[I.in[0]], fr.ptr[I.in[1]], m->d_active, w, M, q.D, q.E, s) != 0) return -1;
      }
      m->moe_last_m = M;
      Prof p(m, "moe_experts");  // the two grouped expert GEMMs
      return launch_moe_experts(fr.ptr[I.in[0]], fr.ptr[I.in[2]], fr.ptr[I.in[3]], w, out, M, q.D, q.H, q.E, s);
    }
    case Op::Binop: {
      const size_t na = fr.numel[I.in[0]];
      if (I.in_group) {  // operator-less binop inside a GEMM group: identity (codegen.cpp:2073-2075)
        fr.numel[I.res] = na;
        fr.ptr[I.res] = fr.ptr[I.in[0]];
        return 0;
      }
      // the raw input as right operand reads the emitted code's never-filled
      // buf_x (codegen.cpp:2014-2016): an empty B, i.e. B = 0
      const size_t nb = I.in[1] == F.x ? 0 : fr.numel[I.in[1]];
      NSH_OUT(c, I.res, na);
      Prof p(m, "binop");
      return launch_binop(fr.ptr[I.in[0]], fr.ptr[I.in[1]], c, (int64_t)na, (int64_t)nb, I.binop, s);
    }
    case Op::Softmax: {
      // rows of: the group's N; train: the input's width (codegen.cpp:2860-2873);
      // else the result's, the input's static columns, or 1 (codegen.cpp:2027-2033)
      int64_t last;
      if (I.in_group) last = I.group_n;
      else if (train) last = F.width[I.in[0]];
      else last = F.scols[I.res] > 0 ? F.scols[I.res] : F.scols[I.in[0]];
      if (last <= 0) last = 1;
      const size_t n = fr.numel[I.in[0]];
      NSH_OUT(y, I.res, n);
      Prof p(m, "softmax");
      return launch_softmax(fr.ptr[I.in[0]], y, (int64_t)n, last, s);
    }
    case Op::Constant: {
      NSH_OUT(y, I.res, 1);
      return launch_fill(y, 1, I.value, s);
    }
    case Op::Reshape:  // a copy of the input's values (codegen.cpp:2124-2128)
      fr.numel[I.res] = fr.numel[I.in[0]];
      fr.ptr[I.res] = fr.ptr[I.in[0]];
      return 0;
    case Op::Transpose: {
      const int64_t C = F.scols[I.in[0]] > 0 ? F.scols[I.in[0]] : 1;
      const size_t n = fr.numel[I.in[0]];
      const int64_t R = F.srows[I.in[0]] > 0 ? F.srows[I.in[0]] : (int64_t)(n / (size_t)C);
      if ((size_t)(R * C) > n) {
        set_error("transpose: static shape exceeds the operand");
        return -1;
      }
      NSH_OUT(y, I.res, (size_t)(R * C));
      Prof p(m, "movement");
      return launch_transpose(fr.ptr[I.in[0]], y, R, C, s);
    }
    case Op::Concat: {
      const size_t na = fr.numel[I.in[0]], nb = fr.numel[I.in[1]];
      Prof p(m, "movement");
      if (I.axis == 0) {  // ns_concat0: rows of a, then rows of b
        const int64_t D = F.scols[I.in[0]] > 0 ? F.scols[I.in[0]] : 1;
        const int64_t ba = (int64_t)(na / (size_t)D), bb = (int64_t)(nb / (size_t)D);
        NSH_OUT(y, I.res, (size_t)((ba + bb) * D));
        if (launch_copy(fr.ptr[I.in[0]], y, ba * D, s) != 0) return -1;
        return launch_copy(fr.ptr[I.in[1]], y + ba * D, bb * D, s);
      }
      const int64_t ca = F.scols[I.in[0]] > 0 ? F.scols[I.in[0]] : 1;
      const int64_t cb = F.scols[I.in[1]] > 0 ? F.scols[I.in[1]] : 1;
      const int64_t R = (int64_t)(na / (size_t)ca);
      if ((size_t)(R * cb) > nb) {
        set_error("concat: the second operand has fewer rows than the first");
        return -1;
      }
      NSH_OUT(y, I.res, (size_t)(R * (ca + cb)));
      return launch_concat_cols(fr.ptr[I.in[0]], fr.ptr[I.in[1]], y, R, ca, cb, s);
    }
    case Op::Slice: {
      const int64_t C = F.scols[I.in[0]] > 0 ? F.scols[I.in[0]] : 1;
      const size_t n = fr.numel[I.in[0]];
      Prof p(m, "movement");
      if (I.axis == 0) {  // rows [start, stop)
        if ((size_t)(I.stop * C) > n) {
          set_error("slice: row range beyond the operand");
          return -1;
        }
        NSH_OUT(y, I.res, (size_t)((I.stop - I.start) * C));
        return launch_copy(fr.ptr[I.in[0]] + I.start * C, y, (I.stop - I.start) * C, s);
      }
      if (I.stop > C) {
        set_error("slice: column range beyond the row width");
        return -1;
      }
      const int64_t M = (int64_t)(n / (size_t)C);
      NSH_OUT(y, I.res, (size_t)(M * (I.stop - I.start)));
      return launch_slice_cols(fr.ptr[I.in[0]], y, M, C, I.start, I.stop - I.start, s);
    }
    case Op::Index: case Op::Scatter: {
      const int64_t C = F.scols[I.in[0]] > 0 ? F.scols[I.in[0]] : 1;
      const size_t n = fr.numel[I.in[0]];
      const int64_t L = (int64_t)I.idx.size();
      const int64_t M = (int64_t)(n / (size_t)C);
      // rows addressed: axis 1 -> columns of each row, axis 0 -> rows
      // (scatter along rows: the operand's static rows, codegen.cpp:2188-2193)
      const int64_t R = I.op == Op::Scatter && I.axis == 0 ? (F.srows[I.in[0]] > 0 ? F.srows[I.in[0]] : 0) : M;
      const int64_t bound = I.axis == 1 ? C : (I.op == Op::Index ? M : R);
      for (int64_t v : I.idx)
        if (v < 0 || v >= bound) {
          set_error(std::string(I.op == Op::Index ? "index" : "scatter") + ": index " + std::to_string(v) +
                    " out of range");
          return -1;
        }
      if (I.op == Op::Scatter) {
        const size_t need = I.axis == 1 ? (size_t)(M * L) : (size_t)(L * C);
        if ((size_t)(R * C) > n || fr.numel[I.in[1]] < need) {
          set_error("scatter: operand or update smaller than its static shape");
          return -1;
        }
      }
      int64_t*& d = m->dev_idx[I.res];
      if (!d && L > 0) {
        NSH_CHECK(hipMalloc(&d, (size_t)L * sizeof(int64_t)));
        NSH_CHECK(hipMemcpy(d, I.idx.data(), (size_t)L * sizeof(int64_t), hipMemcpyHostToDevice));
      }
      Prof p(m, "movement");
      if (I.op == Op::Index) {
        NSH_OUT(y, I.res, (size_t)(I.axis == 1 ? M * L : L * C));
        return launch_index(fr.ptr[I.in[0]], d, y, M, C, L, I.axis == 1 ? 1 : 0, s);
      }
      NSH_OUT(y, I.res, (size_t)(I.axis == 1 ? M * C : R * C));
      return launch_scatter(fr.ptr[I.in[0]], d, fr.ptr[I.in[1]], y, I.axis == 1 ? M : R, C, L, I.axis == 1 ? 1 : 0,
                            s);
    }
    case Op::Dropout: {
      const size_t n = fr.numel[I.in[0]];
      if (!(train && fr.backward)) {  // inference and objective: a copy (codegen.cpp:1999-2005, :2888-2890)
        fr.numel[I.res] = n;
        fr.ptr[I.res] = fr.ptr[I.in[0]];
        return 0;
      }
      // codegen.cpp:2874-2893: keep ~ bernoulli(1 - r) from the context's
      // mt19937, one draw per element in order, on the host exactly as the
      // reference draws it; the device applies m = keep ? 1/(1-r) : 0.
      const double r = dropout_rate(I.rate);
      std::bernoulli_distribution keep(1.0 - r);
      std::vector<uint8_t>& hk = m->drop_keep[I.res];
      hk.resize(n);
      for (size_t i = 0; i < n; i++) hk[i] = keep(m->rng) ? 1 : 0;
      uint8_t* dk = drop_mask(m, I.res, n);
      if (!dk) return -1;
      if (n) NSH_CHECK(hipMemcpyAsync(dk, hk.data(), n, hipMemcpyHostToDevice, s));
      NSH_OUT(y, I.res, n);
      Prof p(m, "dropout");
      return launch_dropout(fr.ptr[I.in[0]], dk, y, (int64_t)n, dropout_scale(r), s);
    }
    default:
      break;
  }
  (void)F;
  set_error("instruction not supported by this build of libnship");
  return -1;
}

int ensure_device_current(ns_model* m);

// direct (optional): the caller's output buffer, which the instruction that
// produces the return value then writes itself (no copy afterwards), unless
// it overlaps the input (out_buf).
int run_forward(ns_model* m, const float* d_x, size_t n_in, float** d_out, size_t* n_out, float* direct = nullptr) {
  if (ensure_device_current(m) != 0) return -1;
  const Plan& P = *m->plan;
  const Func& F = P.fwd;
  Frame fr;
  bind_weights(m, fr);
  fr.numel[F.x] = n_in;
  fr.ptr[F.x] = const_cast<float*>(d_x);
  if (direct && F.ret >= 0 && F.ret != F.x) {
    fr.direct_id = F.ret;
    fr.direct = direct;
    fr.direct_in = d_x;
    fr.direct_in_n = n_in;
  }
  for (const Instr& I : F.ins) {
    if (I.fused_away || I.op == Op::Marker) continue;
    if (exec_forward_op(m, F, I, fr, false) != 0) return -1;
  }
  if (F.ret < 0) {
    keep_frame(m, fr);
    set_error("forward function has no return value");
    return -1;
  }
  *d_out = fr.ptr[F.ret];
  *n_out = fr.numel[F.ret];
  // the caller's buffer is not the model's to read back later
  if (fr.direct_id >= 0 && fr.ptr[F.ret] == direct) fr.ptr[F.ret] = nullptr;
  keep_frame(m, fr);
  return 0;
}


// ---------------------------------------------------------------------------
// Training: forward body, reverse body, optimizer body (emit_train_core,
// codegen.cpp:2755-3157), with these fusions:
//  * CROSS_ENTROPY computes the LOSS_GRAD seed of the same logits in the same
//    pass (one read of logits and labels);
//  * MATMUL_GRAD_A whose only consumer is an ACTIVATION_GRAD applies act'(pre)
//    in the GEMM epilogue;
//  * the five ATTENTION_GRAD_* of one layer come from one backward pass (the
//    reference recomputes the layer for each; the recomputation is
//    deterministic, so one pass yields the same five quantities).
// ---------------------------------------------------------------------------
int uses_of(const Func& F, int id) {
  int u = 0;
  for (auto& J : F.ins)
    for (int v : J.in) u += v == id;
  return u;
}

struct AttnGrads {
  float* dX = nullptr;
  float* dW3 = nullptr;  // [3][D][D] dWq, dWk, dWv
  float* dWo = nullptr;
};

int attention_backward(ns_model* m, Frame& fr, const Instr& I, AttnGrads* out) {
  const Plan& P = *m->plan;
  hipStream_t s = m->stream;
  const int x = I.in[1];
  auto it = fr.attn.find(x);
  if (it == fr.attn.end()) {
    set_error("attention backward without its forward");
    return -1;
  }
  const AttnSaved& sv = it->second;
  const int64_t D = P.vals[I.in[2]].rows, H = I.heads, BS = sv.BS;
  const std::string key = std::to_string(x);
  float* dPre = scratch(m, "ag_dpre" + key, (size_t)(BS * D));
  float* dqkv = scratch(m, "ag_dqkv" + key, (size_t)(3 * BS * D));
  float* delta = scratch(m, "ag_delta" + key, (size_t)(H * BS));
  out->dX = scratch(m, "ag_dx" + key, (size_t)(BS * D));
  out->dW3 = scratch(m, "ag_dw3" + key, (size_t)(3 * D * D));
  out->dWo = scratch(m, "ag_dwo" + key, (size_t)(D * D));
  if (!dPre || !dqkv || !delta || !out->dX || !out->dW3 || !out->dWo) return -1;
  const float* dout = fr.ptr[I.in[0]];
  const float* xin = fr.ptr[x];
  const float* Wq = fr.ptr[I.in[2]];
  const float* Wk = fr.ptr[I.in[3]];
  const float* Wv = fr.ptr[I.in[4]];
  const float* Wo = fr.ptr[I.in[5]];
  if (BS == 0)  // no tokens: every weight gradient is an empty sum
    return launch_fill(out->dW3, 3 * D * D, 0.f, s) != 0 || launch_fill(out->dWo, D * D, 0.f, s) != 0 ? -1 : 0;
  {
    Prof p(m, "gemm");
    // dPre = dout Wo^T
    if (rt_gemm(m, dout, Wo, dPre, BS, D, D, D, D, D, false, true, 0) != 0) return -1;
    // dWo = ctx^T dout
    if (rt_gemm(m, sv.ctx, dout, out->dWo, D, D, BS, D, D, D, true, false, 0) != 0) return -1;
  }
  {
    Prof p(m, "attention_bwd");
    const size_t nds = attention_bwd_ds_floats(BS, D, H);
    float* ds = nds ? scratch(m, "attn_ds", nds) : nullptr;
    if (nds && !ds) return -1;
    const void* rd[5] = {sv.qkv, sv.qkv + BS * D, sv.qkv + 2 * BS * D, sv.ctx, dPre};
    float* pad = nullptr;
    if (!attention_in_place(D, H, D, rd, 5) && !(pad = scratch(m, "attn_pad", attention_pad_floats(BS, D, H, true))))
      return -1;
    if (launch_attention_bwd(sv.qkv, sv.qkv + BS * D, sv.qkv + 2 * BS * D, sv.ctx, dPre, sv.lse, delta, dqkv,
                             dqkv + BS * D, dqkv + 2 * BS * D, BS, D, H, D, ds, pad, s) != 0)
      return -1;
  }
  Prof p(m, "gemm");
  // dWq, dWk, dWv = x^T [dQ | dK | dV]  (one batched launch)
  GemmArgs g;
  g.A = xin; g.B = dqkv; g.C = out->dW3;
  g.M = (int)D; g.N = (int)D; g.K = (int)BS;
  g.lda = D; g.ldb = D; g.ldc = D;
  g.sA = 0; g.sB = BS * D; g.sC = D * D;
  if (rt_gemm_ex(m, g, true, false, 3) != 0) return -1;
  // dX = dQ Wq^T + dK Wk^T + dV Wv^T.  With Wq, Wk, Wv consecutive in the
  // blob: one product over K = 3D, its operands K-blocked ([dQ dK dV] and
  // [Wq Wk Wv], blocks of D), which sums the three products' terms in one
  // chain (c5: 208 us against 73 + 89 + 89 for three launches, the second
  // and third accumulating).  Otherwise three launches.
  const bool packed = Wk == Wq + D * D && Wv == Wk + D * D && D % 16 == 0 &&
                      (reinterpret_cast<uintptr_t>(Wq) | reinterpret_cast<uintptr_t>(dqkv)) % 16 == 0;
  if (packed) {
    GemmArgs h;
    h.A = dqkv; h.B = Wq; h.C = out->dX;
    h.M = (int)BS; h.N = (int)D; h.K = (int)(3 * D);
    h.lda = D; h.ldb = D; h.ldc = D;
    h.kblk = (int)D; h.sAk = BS * D; h.sBk = D * D;
    return rt_gemm_ex(m, h, false, true, 1);
  }
  const float* Ws[3] = {Wq, Wk, Wv};
  for (int j = 0; j < 3; j++) {
    GemmArgs h;
    h.A = dqkv + j * BS * D; h.B = Ws[j]; h.C = out->dX;
    h.M = (int)BS; h.N = (int)D; h.K = (int)D;
    h.lda = D; h.ldb = D; h.ldc = D;
    h.mode = j == 0 ? kEpiAct : kEpiAccum;
    if (rt_gemm_ex(m, h, false, true, 1) != 0) return -1;
  }
  return 0;
}

// Order of the Muon matrices in one step's launches: longest vectors first,
// so that the MGS panel launches dispatch the workgroups with the most work
// per vector before the short ones (each workgroup takes a whole CU), and
// the short matrices fill the CUs that free up.  Each matrix's result does
// not depend on the order.
void order_for_mgs(std::vector<MuonMat>& mats) {
  std::stable_sort(mats.begin(), mats.end(), [](const MuonMat& a, const MuonMat& b) { return a.R > b.R; });
}

// Muon step of several matrices: descriptors to the device, gather, MGS
// column steps, update.
int muon_batch(MuonMat* d, std::vector<MuonMat> mats, int64_t max_elems, hipStream_t s) {
  order_for_mgs(mats);
  const int nm = (int)mats.size();
  NSH_CHECK(hipMemcpyAsync(d, mats.data(), nm * sizeof(MuonMat), hipMemcpyHostToDevice, s));
  if (launch_muon_gather(d, nm, max_elems, s) != 0) return -1;
  if (launch_mgs(d, mats.data(), nm, s) != 0) return -1;
  return launch_muon_update(d, nm, max_elems, s);
}

int optimizer_step(ns_model* m, Frame& fr, const Instr& I, float lr) {
  const Plan& P = *m->plan;
  hipStream_t s = m->stream;
  m->muon_host.clear();
  int64_t max_elems = 0;
  for (size_t k = 0; k + 1 < I.in.size(); k += 2) {
    const int wid = I.in[k], gid = I.in[k + 1];
    const Value& W = P.vals[wid];
    const int64_t r = W.rows, c = W.cols, n = r * c;
    float* w = fr.ptr[wid];
    const float* g = fr.ptr[gid];
    if (!g || fr.numel[gid] < (size_t)n) {
      set_error("optimizer: missing gradient for " + W.name);
      return -1;
    }
    const bool muon = !I.adamw_only && r > 1 && c > 1 && std::min(r, c) >= 8;  // codegen.cpp:3097
    if (muon) {
      MuonMat mm;
      mm.w = w;
      mm.g = g;
      mm.transposed = r < c ? 1 : 0;
      mm.R = (int)(r < c ? c : r);
      mm.C = (int)(r < c ? r : c);
      mm.ldT = mm.R;
      mm.T = scratch(m, "muonT" + std::to_string(wid), (size_t)n);
      // the panel path's row compaction only where it can pay: an embedding
      // gradient with fewer live rows than its vector length's layout needs
      const auto et = fr.emb_tokens.find(gid);
      const bool rows = !mm.transposed && et != fr.emb_tokens.end() && mgs_rows_may_compact(mm.R, et->second);
      const size_t nred = mm.R > mgs_max_panel_len() || rows ? mgs_red_floats(mm.R, mm.C) : 0;
      mm.red = nred ? scratch(m, "muonP" + std::to_string(wid), nred) : nullptr;
      if (!mm.T || (nred && !mm.red)) return -1;
      mm.le = lr * sqrtf((float)std::min(r, c));
      mm.decay = 0.01f * lr;
      m->muon_host.push_back(mm);
      max_elems = std::max(max_elems, n);
    } else {
      auto& st = m->adam[wid];
      if (!st.m) {
        NSH_CHECK(hipMalloc(&st.m, (size_t)n * sizeof(float)));
        NSH_CHECK(hipMalloc(&st.v, (size_t)n * sizeof(float)));
        NSH_CHECK(hipMemsetAsync(st.m, 0, (size_t)n * sizeof(float), s));
        NSH_CHECK(hipMemsetAsync(st.v, 0, (size_t)n * sizeof(float), s));
      }
      st.t += 1;
      const float b1t = 1.f - powf(0.9f, (float)st.t), b2t = 1.f - powf(0.999f, (float)st.t);
      Prof p(m, "adamw");
      if (launch_adamw(w, g, st.m, st.v, n, lr, b1t, b2t, s) != 0) return -1;
    }
  }
  if (m->muon_host.empty()) return 0;
  order_for_mgs(m->muon_host);
  const int nm = (int)m->muon_host.size();
  MuonMat* d = reinterpret_cast<MuonMat*>(scratch(m, "muon_desc", (nm * sizeof(MuonMat) + 3) / 4));
  if (!d) return -1;
  // the three phases as separate profile regions: the transposes are
  // HBM-bound, the MGS launches latency-bound
  NSH_CHECK(hipMemcpyAsync(d, m->muon_host.data(), nm * sizeof(MuonMat), hipMemcpyHostToDevice, s));
  {
    Prof p(m, "muon_gather");
    if (launch_muon_gather(d, nm, max_elems, s) != 0) return -1;
  }
  bool long_vec = false, short_vec = false;
  for (const MuonMat& mm : m->muon_host) (mm.R > mgs_max_panel_len() ? long_vec : short_vec) = true;
  if (long_vec && short_vec && !m->muon_side.stream) {
    NSH_CHECK(hipEventCreateWithFlags(&m->muon_side.fork, hipEventDisableTiming));
    NSH_CHECK(hipEventCreateWithFlags(&m->muon_side.join, hipEventDisableTiming));
    NSH_CHECK(hipStreamCreateWithFlags(&m->muon_side.stream, hipStreamNonBlocking));
  }
  {
    Prof p(m, "muon_mgs");
    if (launch_mgs(d, m->muon_host.data(), nm, s, &m->muon_side) != 0) return -1;
  }
  Prof p(m, "muon_update");
  return launch_muon_update(d, nm, max_elems, s);
}

// Class count of CROSS_ENTROPY / LOSS_GRAD: the logits' static columns
// (result type or weight shape), else the input width, not the propagated
// width (codegen.cpp:2896, :2904); rows = numel / C.
int64_t ce_classes(const Func& F, const Plan& P, int preds) {
  const int64_t c = preds < (int)F.scols.size() ? F.scols[preds] : -1;
  return c > 0 ? c : P.in_cols;
}

// Uploads deferred host labels (a host-pointer train call) on the copy
// stream and makes the model's stream wait for them.  Called by the ops that
// read the labels: the kernels of the forward pass, already enqueued, run
// while the host stages the upload.
int labels_ready(ns_model* m) {
  if (!m->labels_host) return 0;
  const float* host = m->labels_host;
  m->labels_host = nullptr;
  if (!m->copy_stream) NSH_CHECK(hipStreamCreateWithFlags(&m->copy_stream, hipStreamNonBlocking));
  if (!m->labels_ev) NSH_CHECK(hipEventCreateWithFlags(&m->labels_ev, hipEventDisableTiming));
  // work enqueued before this call (which may still read the label buffer)
  // finishes before the upload overwrites it
  NSH_CHECK(hipStreamWaitEvent(m->copy_stream, m->before_ev, 0));
  if (stage_h2d(m->stage, m->labels_dev, host, m->labels_bytes, m->copy_stream) != 0) return -1;
  NSH_CHECK(hipEventRecord(m->labels_ev, m->copy_stream));
  NSH_CHECK(hipStreamWaitEvent(m->stream, m->labels_ev, 0));
  return 0;
}

int run_train(ns_model* m, const float* d_x, size_t n_in, const float* d_y, float lr, bool train_mode,
              float** d_loss) {
  if (ensure_device_current(m) != 0) return -1;
  const Plan& P = *m->plan;
  const Func& F = P.trn;
  hipStream_t s = m->stream;
  Frame fr;
  bind_weights(m, fr);
  fr.backward = train_mode;
  fr.numel[F.x] = n_in;
  fr.ptr[F.x] = const_cast<float*>(d_x);
  float* loss = scratch(m, "loss", 1);
  if (!loss) return -1;
  *d_loss = loss;
  std::map<int, AttnGrads> agrads;
  bool moe_done = false;
  float *moe_dx = nullptr, *moe_dwg = nullptr, *moe_dwe1 = nullptr, *moe_dwe2 = nullptr;
  std::vector<bool> skip(F.ins.size(), false);
  for (size_t ii = 0; ii < F.ins.size(); ii++) {
    const Instr& I = F.ins[ii];
    if (skip[ii] || I.op == Op::Marker) continue;
    switch (I.op) {
      case Op::Matmul: {
        // MATMUL then ACTIVATION of its result: one GEMM writes both the
        // pre-activation (kept for the backward pass) and the activation
        const Instr* J = ii + 1 < F.ins.size() ? &F.ins[ii + 1] : nullptr;
        if (J && J->op == Op::Act && J->in[0] == I.res && I.act == 0 && !I.in_group) {
          const int64_t K = I.k, N = I.n;
          const int64_t M = (int64_t)(fr.numel[I.in[0]] / (size_t)K);
          if (fr.numel[I.in[1]] < (size_t)(K * N) || M > INT32_MAX) {
            set_error("matmul: operand '" + P.vals[I.in[1]].name + "' is smaller than its static shape");
            return -1;
          }
          NSH_OUT(C, I.res, (size_t)(M * N));
          NSH_OUT(Y, J->res, (size_t)(M * N));
          GemmArgs g;
          g.A = fr.ptr[I.in[0]]; g.B = fr.ptr[I.in[1]]; g.C = C; g.C2 = Y;
          g.M = (int)M; g.N = (int)N; g.K = (int)K;
          g.lda = K; g.ldb = N; g.ldc = N;
          g.act = J->act;
          if (fr.backward && J->act == kActRelu) {
            // the backward's relu' reads these bits instead of the
            // pre-activation (4 MB instead of 134 MB at c5)
            // (2 * ceil(M / 32) * N 16-bit values)
            float* bits = scratch(m, "relu_bits" + std::to_string(I.res), (size_t)(ceil_div(M, 32) * N));
            if (!bits) return -1;
            g.mask_out = reinterpret_cast<uint16_t*>(bits);
            g.ldmask = N;
            fr.relu_bits[I.res] = {g.mask_out, N};
          }
          Prof p(m, "gemm");
          if (rt_gemm_ex(m, g, false, false, 1) != 0) return -1;
          skip[ii + 1] = true;
          break;
        }
        if (exec_forward_op(m, F, I, fr, true) != 0) return -1;
        break;
      }
      case Op::Act: case Op::Embedding: case Op::LayerNorm: case Op::Attention: case Op::Moe:
      case Op::Dropout: case Op::Softmax:
        if (exec_forward_op(m, F, I, fr, true) != 0) return -1;
        break;
      case Op::CrossEntropy: {
        const int64_t C = ce_classes(F, P, I.in[0]);
        const size_t n = fr.numel[I.in[0]];
        const int64_t rows = (int64_t)(n / (size_t)C);
        fr.numel[F.y] = n;
        fr.ptr[F.y] = const_cast<float*>(d_y);
        if (labels_ready(m) != 0) return -1;
        float* rl = scratch(m, "row_loss", (size_t)std::max<int64_t>(rows, 1));
        if (!rl) return -1;
        float* grad = nullptr;
        if (train_mode) {
          for (size_t jj = ii + 1; jj < F.ins.size(); jj++) {
            const Instr& J = F.ins[jj];
            if (J.op == Op::LossGrad && J.in[0] == I.in[0] && J.in[1] == I.in[1]) {
              grad = out_buf(m, fr, J.res, n);
              if (!grad) return -1;
              skip[jj] = true;
              break;
            }
          }
        }
        Prof p(m, "softmax_xent");
        if (launch_softmax_xent(fr.ptr[I.in[0]], d_y, grad, rl, loss, rows, C, grad != nullptr, s) != 0) return -1;
        // ns_loss_grad leaves the elements past the last whole row unwritten:
        // zeros in the freshly sized buffer (codegen.cpp:1582-1595)
        if (grad && (size_t)(rows * C) < n && launch_fill(grad + rows * C, (int64_t)n - rows * C, 0.f, s) != 0)
          return -1;
        break;
      }
      default:
        if (!train_mode) break;
        switch (I.op) {
          case Op::LossGrad: {
            const int64_t C = ce_classes(F, P, I.in[0]);
            const size_t n = fr.numel[I.in[0]];
            const int64_t rows = (int64_t)(n / (size_t)C);
            NSH_OUT(grad, I.res, n);
            float* rl = scratch(m, "row_loss", (size_t)std::max<int64_t>(rows, 1));
            float* tmp = scratch(m, "loss_tmp", 1);
            if (!rl || !tmp) return -1;
            if (labels_ready(m) != 0) return -1;
            Prof p(m, "softmax_xent");
            if (launch_softmax_xent(fr.ptr[I.in[0]], d_y, grad, rl, tmp, rows, C, true, s) != 0) return -1;
            if ((size_t)(rows * C) < n && launch_fill(grad + rows * C, (int64_t)n - rows * C, 0.f, s) != 0) return -1;
            break;
          }
          case Op::MatmulGradA: {
            const Value& B = P.vals[I.in[1]];
            const int64_t K = B.rows, N = B.cols;
            const int64_t M = (int64_t)(fr.numel[I.in[0]] / (size_t)N);
            GemmArgs g;
            g.A = fr.ptr[I.in[0]]; g.B = fr.ptr[I.in[1]];
            g.M = (int)M; g.N = (int)K; g.K = (int)N;
            g.lda = N; g.ldb = N; g.ldc = K;
            int res = I.res;
            // the ACTIVATION_GRAD of this result (its only use; a
            // MATMUL_GRAD_W may come first) runs in the GEMM's epilogue
            for (size_t jj = ii + 1; jj < F.ins.size() && uses_of(F, I.res) == 1; jj++) {
              const Instr& J = F.ins[jj];
              if (std::find(J.in.begin(), J.in.end(), I.res) == J.in.end()) continue;
              if (J.op == Op::ActGrad && !J.dropout && J.in[0] == I.res && fr.ptr[J.in[1]]) {
                g.mode = kEpiActGrad;
                g.act = J.act;
                g.aux = fr.ptr[J.in[1]];
                g.ldaux = K;
                auto bits = fr.relu_bits.find(J.in[1]);
                if (J.act == kActRelu && bits != fr.relu_bits.end() && bits->second.second == K) {
                  g.mask_in = bits->second.first;
                  g.ldmask = bits->second.second;
                }
                res = J.res;
                skip[jj] = true;
              }
              break;
            }
            NSH_OUT(C, res, (size_t)(M * K));
            g.C = C;
            Prof p(m, "gemm");
            if (rt_gemm_ex(m, g, false, true, 1) != 0) return -1;
            break;
          }
          case Op::MatmulGradW: {
            const Value& B = P.vals[I.in[2]];
            const int64_t K = B.rows, N = B.cols;
            const int64_t M = (int64_t)(fr.numel[I.in[1]] / (size_t)N);
            NSH_OUT(C, I.res, (size_t)(K * N));
            Prof p(m, "gemm");
            if (rt_gemm(m, fr.ptr[I.in[0]], fr.ptr[I.in[1]], C, K, N, M, K, N, N, true, false, 0) != 0) return -1;
            break;
          }
          case Op::ActGrad: {
            const size_t n = fr.numel[I.in[0]];
            NSH_OUT(y, I.res, n);
            if (I.dropout) {  // dOut * the dropout's saved mask (codegen.cpp:3066-3073)
              if (fr.numel[I.in[1]] != n) {
                set_error("dropout grad: size differs from its forward");
                return -1;
              }
              Prof p(m, "dropout");
              if (launch_dropout(fr.ptr[I.in[0]], drop_mask(m, I.in[1], n), y, (int64_t)n,
                                 dropout_scale(dropout_rate(I.rate)), s) != 0)
                return -1;
              break;
            }
            Prof p(m, "act_grad");
            if (launch_act_grad(fr.ptr[I.in[0]], fr.ptr[I.in[1]], y, (int64_t)n, I.act, s) != 0) return -1;
            break;
          }
          case Op::LayerNormGrad: {
            int64_t last = F.width[I.in[1]];
            if (last <= 0) last = 1;
            const size_t n = fr.numel[I.in[0]];
            NSH_OUT(y, I.res, n);
            Prof p(m, "layernorm_grad");
            if (launch_layernorm_grad(fr.ptr[I.in[0]], fr.ptr[I.in[1]], y, (int64_t)(n / (size_t)last), last, s) != 0)
              return -1;
            break;
          }
          case Op::EmbeddingGradW: {
            const Value& W = P.vals[I.in[2]];
            const int64_t n = (int64_t)(fr.numel[I.in[0]] / (size_t)W.cols);
            NSH_OUT(dW, I.res, (size_t)(W.rows * W.cols));
            int* ws = reinterpret_cast<int*>(scratch(m, "emb_ws", embedding_grad_workspace(n, W.rows)));
            if (!ws) return -1;
            Prof p(m, "embedding_grad");
            if (launch_embedding_grad(fr.ptr[I.in[0]], fr.ptr[I.in[1]], dW, n, W.rows, W.cols, ws, s) != 0)
              return -1;
            fr.emb_tokens[I.res] = n;
            break;
          }
          case Op::AttnGradX: case Op::AttnGradWq: case Op::AttnGradWk: case Op::AttnGradWv: case Op::AttnGradWo: {
            const int x = I.in[1];
            if (!agrads.count(x)) {
              AttnGrads ag;
              if (attention_backward(m, fr, I, &ag) != 0) return -1;
              agrads[x] = ag;
            }
            const AttnGrads& ag = agrads[x];
            const int64_t D = P.vals[I.in[2]].rows;
            const size_t dd = (size_t)(D * D);
            float* p = nullptr;
            size_t n = dd;
            switch (I.op) {
              case Op::AttnGradX: p = ag.dX; n = fr.numel[I.in[0]]; break;
              case Op::AttnGradWq: p = ag.dW3; break;
              case Op::AttnGradWk: p = ag.dW3 + dd; break;
              case Op::AttnGradWv: p = ag.dW3 + 2 * dd; break;
              default: p = ag.dWo; break;
            }
            fr.ptr[I.res] = p;
            fr.numel[I.res] = n;
            break;
          }
          case Op::MoeGradX: case Op::MoeGradWg: case Op::MoeGradWe1: case Op::MoeGradWe2: {
            const MoeInfo& q = P.moe;
            const int64_t M = (int64_t)(fr.numel[I.in[0]] / (size_t)q.D);
            if (!moe_done) {
              MoeWork w;
              if (moe_work(m, M, &w) != 0) return -1;
              w.pre = scratch(m, "moe_pre", (size_t)(M * q.H));
              MoeBwdWork b;
              b.dpre2 = scratch(m, "moe_dpre2", (size_t)(M * q.H));
              b.dH = scratch(m, "moe_dH", (size_t)(M * q.H));
              b.hp = scratch(m, "moe_hp", (size_t)(M * q.H));
              b.dg = scratch(m, "moe_dg", (size_t)(M * q.E));
              b.xs = scratch(m, "moe_xs", (size_t)(M * q.D));
              b.ds = scratch(m, "moe_ds", (size_t)(M * q.D));
              b.splitk_floats = moe_bwd_splitk_floats(M, q.D, q.E);
              b.splitk = b.splitk_floats ? scratch(m, "moe_splitk", b.splitk_floats) : nullptr;
              if (b.splitk_floats && !b.splitk) return -1;
              b.kitems = reinterpret_cast<int*>(scratch(m, "moe_kitems", moe_bwd_kitem_ints(M, q.E)));
              const size_t nkp = moe_bwd_kpart_floats(M, q.D, q.H);
              b.kpart = nkp ? scratch(m, "moe_kpart", nkp) : nullptr;
              if (!b.kitems || (nkp && !b.kpart)) return -1;
              moe_dx = scratch(m, "moe_gx", (size_t)(M * q.D));
              moe_dwg = scratch(m, "moe_gwg", (size_t)(q.D * q.E));
              moe_dwe1 = scratch(m, "moe_gwe1", (size_t)(q.E * q.D * q.H));
              moe_dwe2 = scratch(m, "moe_gwe2", (size_t)(q.E * q.H * q.D));
              if (!w.pre || !b.dpre2 || !b.dH || !b.hp || !b.dg || !b.xs || !b.ds || !moe_dx || !moe_dwg ||
                  !moe_dwe1 || !moe_dwe2)
                return -1;
              // per-expert flags: all set when the flags or either gradient
              // buffer is new (fresh memory holds anything)
              b.dirty = reinterpret_cast<int*>(scratch(m, "moe_dirty", (size_t)q.E));
              if (!b.dirty) return -1;
              if (m->moe_dirty_for[0] != b.dirty || m->moe_dirty_for[1] != moe_dwe1 ||
                  m->moe_dirty_for[2] != moe_dwe2) {
                NSH_CHECK(hipMemsetAsync(b.dirty, 1, (size_t)q.E * sizeof(int), s));
                m->moe_dirty_for[0] = b.dirty;
                m->moe_dirty_for[1] = moe_dwe1;
                m->moe_dirty_for[2] = moe_dwe2;
              }
              // three profile regions: the expert-grouped products (dpre2 and
              // dx), the router gradient, the K-grouped weight gradients
              static const std::pair<const char*, int> kPhases[] = {
                  {"moe_bwd_grouped", kMoeBwdGrouped}, {"moe_bwd_gate", kMoeBwdGate},
                  {"moe_bwd_kgrouped", kMoeBwdKGrouped}};
              for (const auto& ph : kPhases) {
                Prof p(m, ph.first);
                if (launch_moe_backward(fr.ptr[I.in[1]], fr.ptr[I.in[0]], fr.ptr[I.in[2]], fr.ptr[I.in[3]],
                                        fr.ptr[I.in[4]], m->d_active, w, b, moe_dx, moe_dwg, moe_dwe1, moe_dwe2, M,
                                        q.D, q.H, q.E, s, ph.second) != 0)
                  return -1;
              }
              moe_done = true;
            }
            switch (I.op) {
              case Op::MoeGradX: fr.ptr[I.res] = moe_dx; fr.numel[I.res] = (size_t)(M * q.D); break;
              case Op::MoeGradWg: fr.ptr[I.res] = moe_dwg; fr.numel[I.res] = (size_t)(q.D * q.E); break;
              case Op::MoeGradWe1: fr.ptr[I.res] = moe_dwe1; fr.numel[I.res] = (size_t)(q.E * q.D * q.H); break;
              default: fr.ptr[I.res] = moe_dwe2; fr.numel[I.res] = (size_t)(q.E * q.H * q.D); break;
            }
            break;
          }
          case Op::OptStep:
            if (optimizer_step(m, fr, I, lr) != 0) return -1;
            m->host_stale = true;
            break;
          default:
            set_error("training instruction not supported by this build of libnship");
            return -1;
        }
    }
  }
  keep_frame(m, fr);
  return 0;
}

int host_sync_weights(const ns_model* m) {
  if (!m->host_stale) return 0;
  ns_model* mm = const_cast<ns_model*>(m);
  if (stage_d2h(mm->stage, mm->h_w.data(), mm->d_w, mm->h_w.size() * sizeof(float), mm->stream) != 0) return -1;
  mm->host_stale = false;
  return 0;
}

// Host -> device copies of the host blob and the liveness mask.  They are
// enqueued on the model's stream, so kernels still running on it (a
// device-pointer call returns before completion) finish first, and the call
// waits for them because the host vectors may change right after.  A failed
// upload marks the device blob stale; the next device call re-uploads it.
int upload_weights(ns_model* m, size_t off, size_t n) {
  if (n == 0) return 0;
  hipError_t e = hipMemcpyAsync(m->d_w + off, m->h_w.data() + off, n * sizeof(float), hipMemcpyHostToDevice,
                                m->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
  if (e != hipSuccess) {
    m->device_stale = true;
    set_error(std::string("weight upload: ") + hipGetErrorString(e));
    return -1;
  }
  return 0;
}

int upload_mask(ns_model* m) {
  if (!m->d_active || m->moe_active.empty()) return 0;
  hipError_t e = hipMemcpyAsync(m->d_active, m->moe_active.data(), m->moe_active.size(), hipMemcpyHostToDevice,
                                m->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
  if (e != hipSuccess) {
    m->mask_stale = true;  // only the mask: the device weights may be newer than h_w
    set_error(std::string("mask upload: ") + hipGetErrorString(e));
    return -1;
  }
  m->mask_stale = false;
  return 0;
}

int device_sync_weights(ns_model* m) {
  if (upload_weights(m, 0, m->h_w.size()) != 0 || upload_mask(m) != 0) return -1;
  m->device_stale = false;
  return 0;
}

// Before any device work: a lifecycle edit whose upload failed is re-sent
// (the whole blob after a failed weight upload, else only a failed mask).
int ensure_device_current(ns_model* m) {
  if (m->device_stale) return device_sync_weights(m);
  return m->mask_stale ? upload_mask(m) : 0;
}

}  // namespace
}  // namespace nship

// ===========================================================================
// C-ABI
// ===========================================================================
extern "C" {

const char* nsh_last_error(void) { return g_err.c_str(); }

int nsh_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

void* nsh_dev_alloc(size_t bytes) {
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
  if (e != hipSuccess) {
    set_error(std::string("hipMalloc: ") + hipGetErrorString(e));
    return nullptr;
  }
  return p;
}

int nsh_dev_free(void* p) {
  if (p) NSH_CHECK(hipFree(p));
  return 0;
}

// The copies first wait for the whole device: a model's work runs on its own
// non-blocking stream, which a null-stream hipMemcpy would not wait for, so
// a read right after nsh_eval_infer_device / nsh_train_step_device sees the
// finished results (and a write cannot overtake kernels still reading).
int nsh_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  NSH_CHECK(hipDeviceSynchronize());
  NSH_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return 0;
}

int nsh_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  NSH_CHECK(hipDeviceSynchronize());
  NSH_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return 0;
}

int nsh_memset_d(void* dst, int value, size_t bytes) {
  NSH_CHECK(hipMemset(dst, value, bytes));
  return 0;
}

int nsh_device_synchronize(void) {
  NSH_CHECK(hipDeviceSynchronize());
  return 0;
}

// ---- plans -----------------------------------------------------------------
nsh_plan* nsh_plan_parse(const char* ir_text) {
  std::string err;
  Plan* p = parse_plan(ir_text, &err);
  if (!p) {
    set_error("plan: " + err);
    return nullptr;
  }
  nsh_plan* h = new nsh_plan();
  h->p.reset(p);
  return h;
}

void nsh_plan_free(nsh_plan* p) {
  if (p && p->fwd) nsh_model_free(p->fwd);
  delete p;
}
size_t nsh_plan_weight_count(const nsh_plan* p) { return p ? p->p->total : 0; }
const ns_weight_layout* nsh_plan_layout(const nsh_plan* p) { return p ? &p->p->layout : nullptr; }
size_t nsh_plan_output_numel(const nsh_plan* p, size_t input_numel) {
  if (!p) return 0;
  return (size_t)((int64_t)input_numel / p->p->in_cols) * (size_t)p->p->out_cols;
}
int nsh_plan_has_train(const nsh_plan* p) { return p && p->p->has_train ? 1 : 0; }
int nsh_plan_has_moe(const nsh_plan* p) { return p && p->p->moe.present ? 1 : 0; }
size_t nsh_plan_in_cols(const nsh_plan* p) { return p ? (size_t)p->p->in_cols : 0; }
size_t nsh_plan_out_cols(const nsh_plan* p) { return p ? (size_t)p->p->out_cols : 0; }

// ---- models ----------------------------------------------------------------
void nsh_model_free(ns_model* m);

ns_model* nsh_model_init(const nsh_plan* ph, const float* weights, size_t num_floats) {
  if (!ph || !weights) {
    set_error("init: null plan or weights");
    return nullptr;
  }
  const Plan& P = *ph->p;
  if (num_floats != P.total) {
    set_error("init: weight count mismatch");
    return nullptr;
  }
  ns_model* m = new ns_model();
  m->plan = &P;
  m->arena.resize(P.vals.size());
  bool ok = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) == hipSuccess;
  ok = ok && hipMalloc(&m->d_w, (P.total ? P.total : 1) * sizeof(float)) == hipSuccess;
  if (ok) {
    m->h_w.assign(weights, weights + P.total);
    ok = hipMemcpy(m->d_w, weights, P.total * sizeof(float), hipMemcpyHostToDevice) == hipSuccess;
  }
  if (ok && P.moe.present) {
    m->moe_active.assign((size_t)P.moe.E, 0);
    for (int64_t e = 0; e < P.moe.K0; e++) m->moe_active[(size_t)e] = 1;
    m->moe_count = (size_t)P.moe.K0;
    ok = hipMalloc(&m->d_active, (size_t)P.moe.E) == hipSuccess &&
         hipMemcpy(m->d_active, m->moe_active.data(), (size_t)P.moe.E, hipMemcpyHostToDevice) == hipSuccess;
  }
  if (!ok) {
    set_error("init: device allocation or copy failed");
    nsh_model_free(m);
    return nullptr;
  }
  return m;
}

void nsh_model_free(ns_model* m) {
  if (!m) return;
  if (m->stream) hipStreamSynchronize(m->stream);
  if (m->copy_stream) hipStreamSynchronize(m->copy_stream);
  stage_free(m->stage);
  if (m->labels_ev) hipEventDestroy(m->labels_ev);
  if (m->before_ev) hipEventDestroy(m->before_ev);
  if (m->copy_stream) hipStreamDestroy(m->copy_stream);
  if (m->muon_side.stream) {
    hipStreamSynchronize(m->muon_side.stream);
    hipStreamDestroy(m->muon_side.stream);
  }
  if (m->muon_side.fork) hipEventDestroy(m->muon_side.fork);
  if (m->muon_side.join) hipEventDestroy(m->muon_side.join);
  for (auto& b : m->arena) if (b.p) hipFree(b.p);
  for (auto& kv : m->scratch) if (kv.second.p) hipFree(kv.second.p);
  for (auto& kv : m->dev_idx) if (kv.second) hipFree(kv.second);
  for (auto& e : m->pending) { hipEventDestroy(e.a); hipEventDestroy(e.b); }
  for (auto e : m->event_pool) hipEventDestroy(e);
  if (m->d_w) hipFree(m->d_w);
  if (m->d_active) hipFree(m->d_active);
  for (auto& kv : m->adam) {
    if (kv.second.m) hipFree(kv.second.m);
    if (kv.second.v) hipFree(kv.second.v);
  }
  if (m->stream) hipStreamDestroy(m->stream);
  delete m;
}

int nsh_eval_infer_device(ns_model* m, const float* d_input, float* d_output, size_t input_numel) {
  if (!m || !d_input || !d_output) {
    set_error("eval: null argument");
    return -1;
  }
  float* res = nullptr;
  size_t n = 0;
  if (run_forward(m, d_input, input_numel, &res, &n, d_output) != 0) return -1;
  if (n && res != d_output)
    NSH_CHECK(hipMemcpyAsync(d_output, res, n * sizeof(float), hipMemcpyDeviceToDevice, m->stream));
  return 0;
}

int nsh_model_sync(ns_model* m) {
  if (!m) return -1;
  return sync(m);
}

int nsh_eval_infer(ns_model* m, const float* input, float* output, size_t input_numel) {
  if (!m || !input || !output) {
    set_error("eval: null argument");
    return -1;
  }
  Buf& xb = m->scratch["__x"];
  if (ensure(xb, input_numel) != 0) return -1;
  if (stage_h2d(m->stage, xb.p, input, input_numel * sizeof(float), m->stream) != 0) return -1;
  float* res = nullptr;
  size_t n = 0;
  if (run_forward(m, xb.p, input_numel, &res, &n) != 0) return -1;
  if (n && stage_d2h(m->stage, output, res, n * sizeof(float), m->stream) != 0) return -1;
  return sync(m);
}

size_t nsh_model_weight_count(const ns_model* m) { return m ? m->plan->total : 0; }

int nsh_model_get_weights(const ns_model* m, float* out, size_t n) {
  if (!m || !out || n != m->plan->total) return -1;
  if (host_sync_weights(m) != 0) return -1;
  std::memcpy(out, m->h_w.data(), n * sizeof(float));
  return 0;
}

// NSM2 checkpoint: u32 magic, u64 count, f32[count], and for MoE models
// u32 n_layers = 1, u64 capacity, u8[capacity] liveness mask
// (codegen.cpp:2505-2528).
int nsh_save_checkpoint(const ns_model* m, const char* path) {
  if (!m || !path) return -1;
  if (host_sync_weights(m) != 0) return -1;
  FILE* fp = std::fopen(path, "wb");
  if (!fp) return -1;
  const uint32_t magic = 0x4E534D32u;
  const uint64_t count = m->plan->total;
  bool ok = std::fwrite(&magic, sizeof(magic), 1, fp) == 1 && std::fwrite(&count, sizeof(count), 1, fp) == 1 &&
            std::fwrite(m->h_w.data(), sizeof(float), count, fp) == count;
  if (ok && m->plan->moe.present) {
    const uint32_t layers = 1;
    const uint64_t cap = (uint64_t)m->plan->moe.E;
    ok = std::fwrite(&layers, sizeof(layers), 1, fp) == 1 && std::fwrite(&cap, sizeof(cap), 1, fp) == 1 &&
         std::fwrite(m->moe_active.data(), 1, cap, fp) == cap;
  }
  ok = (std::fclose(fp) == 0) && ok;
  return ok ? 0 : -1;
}

// NSM1 (weights only, every expert alive) or NSM2; re-uploads the blob and
// the mask (codegen.cpp:2529-2557 host side, :1032-1034 device re-sync).
// The file is validated completely before the model is touched.
int nsh_load_checkpoint(ns_model* m, const char* path) {
  if (!m || !path) return -1;
  FILE* fp = std::fopen(path, "rb");
  if (!fp) return -1;
  uint32_t magic = 0;
  uint64_t count = 0;
  std::vector<float> w;
  std::vector<uint8_t> mask;
  bool ok = std::fread(&magic, sizeof(magic), 1, fp) == 1 && std::fread(&count, sizeof(count), 1, fp) == 1 &&
            (magic == 0x4E534D31u || magic == 0x4E534D32u) && count == m->plan->total;
  if (ok) {
    w.resize(count);
    ok = std::fread(w.data(), sizeof(float), count, fp) == count;
  }
  if (ok && m->plan->moe.present) {
    const size_t cap_expected = (size_t)m->plan->moe.E;
    if (magic == 0x4E534D32u) {
      uint32_t layers = 0;
      uint64_t cap = 0;
      ok = std::fread(&layers, sizeof(layers), 1, fp) == 1 && std::fread(&cap, sizeof(cap), 1, fp) == 1 &&
           layers == 1 && cap == cap_expected;
      if (ok) {
        mask.resize(cap);
        ok = std::fread(mask.data(), 1, cap, fp) == cap;
      }
    } else {
      mask.assign(cap_expected, 1);
    }
  }
  std::fclose(fp);
  if (!ok) return -1;
  if (sync(m) != 0) return -1;
  m->h_w.swap(w);
  m->host_stale = false;
  if (m->plan->moe.present) {
    m->moe_active.swap(mask);
    m->moe_count = 0;
    for (uint8_t v : m->moe_active) m->moe_count += v;
  }
  return device_sync_weights(m);
}

// ---- MoE lifecycle: host blob edits + device re-sync (codegen.cpp:2562-2626)
size_t nsh_expert_count(const ns_model* m) { return m ? m->moe_count : 0; }

size_t nsh_expert_birth(ns_model* m, int n) {
  if (!m) return 0;
  const MoeInfo& q = m->plan->moe;
  if (!q.present || n <= 0 || m->moe_count >= (size_t)q.E) return m->moe_count;
  if (host_sync_weights(m) != 0) return m->moe_count;
  const size_t cap = (size_t)q.E, D = (size_t)q.D, H = (size_t)q.H;
  const size_t og = m->plan->vals[q.g].offset, o1 = m->plan->vals[q.e1].offset, o2 = m->plan->vals[q.e2].offset;
  float* w = m->h_w.data();
  int src = (int)(m->rng() % cap);
  size_t tries = 0;
  while (tries++ < cap && !m->moe_active[(size_t)src]) src = (int)(m->rng() % cap);
  const size_t s1 = (size_t)src * D * H, s2 = (size_t)src * H * D;
  for (int e = 0; e < (int)cap && n > 0; e++) {
    if (m->moe_active[(size_t)e]) continue;
    const size_t g2 = (size_t)e * D * H, g3 = (size_t)e * H * D;
    for (size_t k = 0; k < D; k++)
      w[og + k * cap + (size_t)e] = w[og + k * cap + (size_t)src] + ((float)(m->rng() % 1001) / 1000.f - 0.5f) * 1e-2f;
    for (size_t t = 0; t < D * H; t++)
      w[o1 + g2 + t] = w[o1 + s1 + t] + ((float)(m->rng() % 1001) / 1000.f - 0.5f) * 1e-2f;
    for (size_t t = 0; t < H * D; t++)
      w[o2 + g3 + t] = w[o2 + s2 + t] + ((float)(m->rng() % 1001) / 1000.f - 0.5f) * 1e-2f;
    m->moe_active[(size_t)e] = 1;
    m->moe_count++;
    n--;
    if (upload_weights(m, o1 + g2, D * H) != 0 || upload_weights(m, o2 + g3, H * D) != 0) return m->moe_count;
  }
  // (a failed upload leaves device_stale or mask_stale set: the next device
  // call retries)
  if (upload_weights(m, og, D * cap) == 0) upload_mask(m);
  return m->moe_count;
}

size_t nsh_expert_merge(ns_model* m, int a, int b) {
  if (!m) return 0;
  const MoeInfo& q = m->plan->moe;
  if (!q.present || a < 0 || b < 0 || a == b || a >= (int)q.E || b >= (int)q.E ||
      !m->moe_active[(size_t)a] || !m->moe_active[(size_t)b])
    return m->moe_count;
  if (host_sync_weights(m) != 0) return m->moe_count;
  const size_t cap = (size_t)q.E, D = (size_t)q.D, H = (size_t)q.H;
  const size_t og = m->plan->vals[q.g].offset, o1 = m->plan->vals[q.e1].offset, o2 = m->plan->vals[q.e2].offset;
  float* w = m->h_w.data();
  for (size_t k = 0; k < D; k++)
    w[og + k * cap + (size_t)a] = 0.5f * (w[og + k * cap + (size_t)a] + w[og + k * cap + (size_t)b]);
  for (size_t t = 0; t < D * H; t++)
    w[o1 + (size_t)a * D * H + t] = 0.5f * (w[o1 + (size_t)a * D * H + t] + w[o1 + (size_t)b * D * H + t]);
  for (size_t t = 0; t < H * D; t++)
    w[o2 + (size_t)a * H * D + t] = 0.5f * (w[o2 + (size_t)a * H * D + t] + w[o2 + (size_t)b * H * D + t]);
  m->moe_active[(size_t)b] = 0;
  m->moe_count--;
  if (upload_weights(m, og, D * cap) == 0 && upload_weights(m, o1 + (size_t)a * D * H, D * H) == 0 &&
      upload_weights(m, o2 + (size_t)a * H * D, H * D) == 0)
    upload_mask(m);
  return m->moe_count;
}

size_t nsh_expert_kill(ns_model* m, int k) {
  if (!m) return 0;
  const MoeInfo& q = m->plan->moe;
  if (!q.present || k < 0 || k >= (int)q.E || !m->moe_active[(size_t)k]) return m->moe_count;
  // only the mask changes (codegen.cpp:2619-2626): the weights stay as
  // they are on the device (the host copy may be older than them)
  m->moe_active[(size_t)k] = 0;
  m->moe_count--;
  upload_mask(m);
  return m->moe_count;
}

// Training step: the wrapper of codegen.cpp:2636-2644 -- the plan's LR
// schedule multiplier at the model's step counter (post-incremented,
// saturating); the reference compiles the constant schedule (multiplier 1).
int nsh_train_step_device(ns_model* m, const float* d_input, const float* d_labels, size_t input_numel,
                          float* loss_out, float lr) {
  if (!m || !d_input || !d_labels) {
    set_error("train: null argument");
    return -1;
  }
  if (!m->plan->has_train) {
    set_error("train: the network has no train() method");
    return -1;
  }
  const int64_t st = m->lr_step;
  if (st < INT64_MAX) m->lr_step = st + 1;
  const float lr_eff = lr * lr_scale(m->plan->lr, st);
  float* d_loss = nullptr;
  if (run_train(m, d_input, input_numel, d_labels, lr_eff, true, &d_loss) != 0) return -1;
  if (loss_out) {
    NSH_CHECK(hipMemcpyAsync(loss_out, d_loss, sizeof(float), hipMemcpyDeviceToHost, m->stream));
    return sync(m);
  }
  return 0;
}

static int stage_train_inputs(ns_model* m, const float* input, const float* labels, size_t input_numel,
                              float** dx, float** dy) {
  const Plan& P = *m->plan;
  const size_t rows = (size_t)((int64_t)input_numel / P.in_cols);
  const size_t ny = rows * (size_t)P.out_cols;
  Buf& xb = m->scratch["__x"];
  Buf& yb = m->scratch["__y"];
  if (ensure(xb, input_numel) != 0 || ensure(yb, ny) != 0) return -1;
  if (!m->before_ev) NSH_CHECK(hipEventCreateWithFlags(&m->before_ev, hipEventDisableTiming));
  NSH_CHECK(hipEventRecord(m->before_ev, m->stream));
  if (stage_h2d(m->stage, xb.p, input, input_numel * sizeof(float), m->stream) != 0) return -1;
  // the labels follow when the loss needs them (labels_ready)
  m->labels_host = labels;
  m->labels_dev = yb.p;
  m->labels_bytes = ny * sizeof(float);
  *dx = xb.p;
  *dy = yb.p;
  return 0;
}

int nsh_train_step(ns_model* m, const float* input, const float* labels, size_t input_numel, float* loss_out,
                   float lr) {
  if (!m || !input || !labels) {
    set_error("train: null argument");
    return -1;
  }
  float *dx = nullptr, *dy = nullptr;
  if (stage_train_inputs(m, input, labels, input_numel, &dx, &dy) != 0) return -1;
  float loss = 0.f;
  const int rc = nsh_train_step_device(m, dx, dy, input_numel, &loss, lr);
  m->labels_host = nullptr;  // not read by this plan, or consumed
  if (rc != 0) return -1;
  if (loss_out) *loss_out = loss;
  return 0;
}

int nsh_objective_loss(ns_model* m, const float* input, const float* labels, size_t input_numel,
                       float* loss_out) {
  if (!m || !input || !labels) {
    set_error("objective: null argument");
    return -1;
  }
  if (!m->plan->has_train) {
    set_error("objective: the network has no train() method");
    return -1;
  }
  float *dx = nullptr, *dy = nullptr;
  if (stage_train_inputs(m, input, labels, input_numel, &dx, &dy) != 0) return -1;
  float* d_loss = nullptr;
  const int rc = run_train(m, dx, input_numel, dy, 0.f, false, &d_loss);
  m->labels_host = nullptr;
  if (rc != 0) return -1;
  float loss = 0.f;
  NSH_CHECK(hipMemcpyAsync(&loss, d_loss, sizeof(float), hipMemcpyDeviceToHost, m->stream));
  if (sync(m) != 0) return -1;
  if (loss_out) *loss_out = loss;
  return 0;
}

float nsh_plan_lr_scale(const nsh_plan* p, int64_t step) { return p ? lr_scale(p->p->lr, step) : 1.0f; }

// ---- stateless entry points of the emitted TU --------------------------------
int nsh_model_set_weights(ns_model* m, const float* w, size_t n) {
  if (!m || !w || n != m->plan->total) {
    set_error("set_weights: null argument or weight count mismatch");
    return -1;
  }
  if (sync(m) != 0) return -1;  // kernels of an earlier device-pointer call read the blob
  std::memcpy(m->h_w.data(), w, n * sizeof(float));
  m->host_stale = false;
  return device_sync_weights(m);
}

int nsh_model_set_expert_mask(ns_model* m, const uint8_t* active) {
  if (!m) return -1;
  const MoeInfo& q = m->plan->moe;
  if (!q.present) return 0;
  if (sync(m) != 0) return -1;
  size_t live = 0;
  for (int64_t e = 0; e < q.E; e++) {
    m->moe_active[(size_t)e] = (!active || active[e] != 0) ? 1 : 0;
    live += m->moe_active[(size_t)e];
  }
  m->moe_count = live;
  return upload_mask(m);
}

// The emitted TU's `forward` (codegen.cpp:2263-2288): the weights come with
// every call, and every call reads them (the reference re-assigns its
// per-weight buffers from `weights`); moe_active NULL = every expert live
// (ns_moe_fwd's `active == NULL`).  One cached model per plan holds the
// device state; like the reference's static buffers it serves one call at a
// time.
int nsh_forward(const nsh_plan* p, const float* input, const float* weights, float* output, size_t input_numel,
                const uint8_t* moe_active) {
  if (!p || !input || !weights || !output) {
    set_error("forward: null argument");
    return -1;
  }
  nsh_plan* ph = const_cast<nsh_plan*>(p);
  if (!ph->fwd) {
    ph->fwd = nsh_model_init(p, weights, p->p->total);
    if (!ph->fwd) return -1;
  } else if (nsh_model_set_weights(ph->fwd, weights, p->p->total) != 0) {
    return -1;
  }
  if (nsh_model_set_expert_mask(ph->fwd, moe_active) != 0) return -1;
  return nsh_eval_infer(ph->fwd, input, output, input_numel);
}

// The emitted TU's `ns_train_core` (codegen.cpp:2753-3157): weights read from
// `w`, one forward (+ backward and optimizer step at `lr` as given when
// train_mode) over the model's context, the loss to *loss_out, and with
// train_mode the updated weights to `wout` (NULL: not written back).  No LR
// schedule and no step counter: those belong to the wrapper.
int nsh_train_core(ns_model* m, const float* x, size_t nx, const float* y, const float* w, float* wout,
                   float* loss_out, float lr, int train_mode) {
  if (!m || !x || !y || !w) {
    set_error("train_core: null argument");
    return -1;
  }
  if (!m->plan->has_train) {
    set_error("train_core: the network has no train() method");
    return -1;
  }
  if (nsh_model_set_weights(m, w, m->plan->total) != 0) return -1;
  float *dx = nullptr, *dy = nullptr;
  if (stage_train_inputs(m, x, y, nx, &dx, &dy) != 0) return -1;
  float* d_loss = nullptr;
  const int rc = run_train(m, dx, nx, dy, train_mode ? lr : 0.f, train_mode != 0, &d_loss);
  m->labels_host = nullptr;
  if (rc != 0) return -1;
  float loss = 0.f;
  NSH_CHECK(hipMemcpyAsync(&loss, d_loss, sizeof(float), hipMemcpyDeviceToHost, m->stream));
  if (sync(m) != 0) return -1;
  if (loss_out) *loss_out = loss;
  if (train_mode && wout && nsh_model_get_weights(m, wout, m->plan->total) != 0) return -1;
  return 0;
}

// ---- profiling ---------------------------------------------------------------
int nsh_profile_enable(ns_model* m, int on) {
  if (!m) return -1;
  if (sync(m) != 0) return -1;
  m->prof = on != 0;
  return 0;
}

int nsh_profile_select(ns_model* m, const char* regions) {
  if (!m) return -1;
  if (sync(m) != 0) return -1;
  m->prof_sel.clear();
  if (!regions) return 0;
  std::string cur;
  for (const char* c = regions;; c++) {
    if (*c == ',' || *c == 0) {
      if (!cur.empty()) m->prof_sel.push_back(cur);
      cur.clear();
      if (!*c) break;
    } else {
      cur += *c;
    }
  }
  return 0;
}

int nsh_profile_reset(ns_model* m) {
  if (!m) return -1;
  if (sync(m) != 0) return -1;
  m->prof_acc.clear();
  return 0;
}

int nsh_profile_report(ns_model* m, char* buf, size_t len) {
  if (!m || !buf || !len) return -1;
  if (sync(m) != 0) return -1;
  std::string s = "{";
  bool first = true;
  for (auto& kv : m->prof_acc) {
    char tmp[256];
    std::snprintf(tmp, sizeof tmp, "%s\"%s\": {\"calls\": %ld, \"ms\": %.6f}", first ? "" : ", ",
                  kv.first.c_str(), kv.second.first, kv.second.second);
    s += tmp;
    first = false;
  }
  s += "}";
  if (s.size() + 1 > len) return -1;
  std::memcpy(buf, s.c_str(), s.size() + 1);
  return 0;
}

// Contents of IR value `name` as left by the last forward / training call
// (weights: their current values).  n must equal the value's element count.
int nsh_model_read_value(ns_model* m, const char* name, float* out, size_t n) {
  if (!m || !name || !out) return -1;
  auto it = m->plan->index.find(name);
  if (it == m->plan->index.end()) {
    set_error(std::string("read_value: no value named ") + name);
    return -1;
  }
  const int id = it->second;
  if (sync(m) != 0) return -1;
  const float* p = nullptr;
  size_t cnt = 0;
  if (m->plan->vals[id].weight) {
    p = m->d_w + m->plan->vals[id].offset;
    cnt = (size_t)(m->plan->vals[id].rows * m->plan->vals[id].cols);
  } else if ((size_t)id < m->last_ptr.size()) {
    p = m->last_ptr[id];
    cnt = m->last_numel[id];
  }
  if (!p || cnt != n) {
    set_error(std::string("read_value: ") + name + " not available with that size");
    return -1;
  }
  NSH_CHECK(hipMemcpy(out, p, n * sizeof(float), hipMemcpyDeviceToHost));
  return 0;
}

int nsh_model_last_routing(ns_model* m, int32_t* best, float* prob, float* logits, size_t n) {
  if (!m || !m->plan->moe.present || (size_t)m->moe_last_m != n) {
    set_error("routing: no MoE forward of that size");
    return -1;
  }
  if (sync(m) != 0) return -1;
  const int64_t E = m->plan->moe.E;
  MoeWork w;
  if (moe_work(m, (int64_t)n, &w) != 0) return -1;
  if (best) NSH_CHECK(hipMemcpy(best, w.best, n * sizeof(int32_t), hipMemcpyDeviceToHost));
  if (prob) NSH_CHECK(hipMemcpy(prob, w.prob, n * sizeof(float), hipMemcpyDeviceToHost));
  if (logits) NSH_CHECK(hipMemcpy(logits, w.logits, n * (size_t)E * sizeof(float), hipMemcpyDeviceToHost));
  return 0;
}

// ---- kernels on device pointers ----------------------------------------------
int nsh_op_gemm(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                int64_t ldb, int64_t ldc, int transA, int transB, int act) {
  if (!A || !B || !C || M < 0 || N < 0 || K < 0) {
    set_error("gemm: bad arguments");
    return -1;
  }
  if (launch_gemm(A, B, C, M, N, K, lda, ldb, ldc, transA != 0, transB != 0, act, nullptr) != 0) return -1;
  NSH_CHECK(hipStreamSynchronize(nullptr));
  return 0;
}

static GemmArgs plain_gemm(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                           int64_t ldb, int64_t ldc, int act) {
  GemmArgs g;
  g.A = A; g.B = B; g.C = C;
  g.M = (int)M; g.N = (int)N; g.K = (int)K;
  g.lda = lda; g.ldb = ldb; g.ldc = ldc;
  g.act = act;
  return g;
}

static int split_of(int64_t M, int64_t N, int64_t K, int splits) {
  if (splits > 0) return splits;
  return gemm_split_count(plain_gemm(nullptr, nullptr, nullptr, M, N, K, 0, 0, 0, 0), 1);
}

size_t nsh_op_gemm_splitk_workspace(int64_t M, int64_t N, int64_t K, int splits) {
  if (M <= 0 || N <= 0 || K < 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return 0;
  const int sp = split_of(M, N, K, splits);
  return gemm_split_workspace(plain_gemm(nullptr, nullptr, nullptr, M, N, K, 0, 0, 0, 0), 1, sp) * sizeof(float);
}

int nsh_op_gemm_splitk(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                       int64_t ldb, int64_t ldc, int transA, int transB, int act, int splits, void* workspace) {
  if (!A || !B || !C || M < 0 || N < 0 || K < 0 || splits < 0 || M > INT32_MAX || N > INT32_MAX ||
      K > INT32_MAX) {
    set_error("gemm_splitk: bad arguments");
    return -1;
  }
  const int sp = split_of(M, N, K, splits);
  if (sp > 1 && !workspace) {
    set_error("gemm_splitk: missing workspace");
    return -1;
  }
  const GemmArgs g = plain_gemm(A, B, C, M, N, K, lda, ldb, ldc, act);
  if (launch_gemm_split(g, transA != 0, transB != 0, 1, sp, (float*)workspace, nullptr) != 0) return -1;
  NSH_CHECK(hipStreamSynchronize(nullptr));
  return 0;
}

#define NSH_OP_DONE()                             \
  do {                                            \
    NSH_CHECK(hipStreamSynchronize(nullptr));     \
    return 0;                                     \
  } while (0)

// Argument checks of the op entry points, before any device work: a null
// buffer that a nonempty call would touch, or a negative size, is an error.
#define NSH_OP_REQUIRE(cond, what)                          \
  do {                                                      \
    if (!(cond)) {                                          \
      set_error(std::string(what) + ": bad arguments");     \
      return -1;                                            \
    }                                                       \
  } while (0)

int nsh_op_embedding(const float* W, const float* idx, float* out, int64_t n, int64_t V, int64_t D) {
  NSH_OP_REQUIRE(n >= 0 && D >= 0 && (n == 0 || D == 0 || (W && idx && out && V > 0)), "embedding");
  if (launch_embedding(W, idx, out, n, V, D, nullptr) != 0) return -1;
  NSH_OP_DONE();
}

int nsh_op_layernorm(const float* x, float* y, int64_t rows, int64_t last) {
  NSH_OP_REQUIRE(rows >= 0 && (rows == 0 || (x && y)), "layernorm");
  if (last <= 0 || launch_layernorm(x, y, rows, last, nullptr) != 0) return -1;
  NSH_OP_DONE();
}

int nsh_op_layernorm_grad(const float* dout, const float* x, float* dx, int64_t rows, int64_t last) {
  NSH_OP_REQUIRE(rows >= 0 && (rows == 0 || (dout && x && dx)), "layernorm_grad");
  if (last <= 0 || launch_layernorm_grad(dout, x, dx, rows, last, nullptr) != 0) return -1;
  NSH_OP_DONE();
}

int nsh_op_softmax_xent(const float* logits, const float* labels, float* grad, float* row_loss, float* loss,
                        int64_t rows, int64_t C) {
  NSH_OP_REQUIRE(rows <= 0 || (logits && labels && row_loss && loss && C > 0), "softmax_xent");
  if (launch_softmax_xent(logits, labels, grad, row_loss, loss, rows, C, grad != nullptr, nullptr) != 0) return -1;
  NSH_OP_DONE();
}

int nsh_op_act_grad(const float* din, const float* pre, float* dout, int64_t n, int act) {
  NSH_OP_REQUIRE(n >= 0 && (n == 0 || (din && pre && dout)), "act_grad");
  if (launch_act_grad(din, pre, dout, n, act, nullptr) != 0) return -1;
  NSH_OP_DONE();
}

size_t nsh_op_embedding_grad_workspace(int64_t n, int64_t V) { return embedding_grad_workspace(n, V) * sizeof(int); }

int nsh_op_embedding_grad(const float* dout, const float* idx, float* dW, int64_t n, int64_t V, int64_t D,
                          void* workspace) {
  NSH_OP_REQUIRE(n >= 0 && V >= 0 && D >= 0 && (V * D == 0 || dW) && (n == 0 || (dout && idx)), "embedding_grad");
  if (V == 0 || D == 0) return 0;  // dW is empty: no device work
  if (!workspace || launch_embedding_grad(dout, idx, dW, n, V, D, (int*)workspace, nullptr) != 0) return -1;
  NSH_OP_DONE();
}

// One Muon matrix on device buffers: w -= lr sqrt(min(r,c)) MGS(g) + 0.01 lr w.
// With w zeroed, lr = -1 and decay 0 it returns MGS(g) itself (orthonormalize).
static int op_muon(float* w, const float* g, int64_t r, int64_t c, float le, float decay, void* ws) {
  if (!w || !g || !ws || r <= 0 || c <= 0) {
    set_error("muon: bad arguments");
    return -1;
  }
  MuonMat mm;
  mm.w = w;
  mm.g = g;
  mm.transposed = r < c ? 1 : 0;
  mm.R = (int)(r < c ? c : r);
  mm.C = (int)(r < c ? r : c);
  mm.ldT = mm.R;
  char* base = (char*)ws;
  mm.T = (float*)(base + 256);
  mm.red = mgs_red_floats(mm.R, mm.C) ? mm.T + r * c : nullptr;
  mm.le = le;
  mm.decay = decay;
  MuonMat* d = (MuonMat*)base;
  NSH_CHECK(hipMemcpy(d, &mm, sizeof(mm), hipMemcpyHostToDevice));
  if (launch_muon_gather(d, 1, r * c, nullptr) != 0) return -1;
  if (launch_mgs(d, &mm, 1, nullptr) != 0) return -1;
  if (launch_muon_update(d, 1, r * c, nullptr) != 0) return -1;
  NSH_CHECK(hipStreamSynchronize(nullptr));
  return 0;
}

int nsh_op_muon_multi(int n, float* const* w, const float* const* g, const int64_t* r, const int64_t* c, float lr,
                      void* workspace) {
  if (n <= 0 || !w || !g || !r || !c || !workspace) {
    set_error("muon_multi: bad arguments");
    return -1;
  }
  std::vector<MuonMat> mats;
  char* base = (char*)workspace;
  MuonMat* d = (MuonMat*)base;
  float* wsf = (float*)(base + 256 * (((size_t)n * sizeof(MuonMat) + 255) / 256));
  int64_t max_elems = 0;
  for (int i = 0; i < n; i++) {
    MuonMat mm;
    mm.w = w[i];
    mm.g = g[i];
    mm.transposed = r[i] < c[i] ? 1 : 0;
    mm.R = (int)(r[i] < c[i] ? c[i] : r[i]);
    mm.C = (int)(r[i] < c[i] ? r[i] : c[i]);
    mm.ldT = mm.R;
    mm.T = wsf;
    wsf += r[i] * c[i];
    const size_t nred = mgs_red_floats(mm.R, mm.C);
    mm.red = nred ? wsf : nullptr;
    wsf += nred;
    mm.le = lr * sqrtf((float)std::min(r[i], c[i]));
    mm.decay = 0.01f * lr;
    mats.push_back(mm);
    max_elems = std::max(max_elems, r[i] * c[i]);
  }
  if (muon_batch(d, mats, max_elems, nullptr) != 0) return -1;
  NSH_CHECK(hipStreamSynchronize(nullptr));
  return 0;
}

size_t nsh_op_muon_multi_workspace(int n, const int64_t* r, const int64_t* c) {
  size_t b = 256 * (((size_t)n * sizeof(MuonMat) + 255) / 256);
  for (int i = 0; i < n; i++)
    b += (size_t)(r[i] * c[i] + (int64_t)mgs_red_floats(std::max(r[i], c[i]), std::min(r[i], c[i]))) * sizeof(float);
  return b;
}

size_t nsh_op_muon_workspace(int64_t r, int64_t c) {
  return 256 + (size_t)(r * c + (int64_t)mgs_red_floats(std::max(r, c), std::min(r, c))) * sizeof(float);
}

int nsh_op_orthonormalize(const float* g, float* q, int64_t r, int64_t c, void* workspace) {
  NSH_CHECK(hipMemset(q, 0, (size_t)(r * c) * sizeof(float)));
  return op_muon(q, g, r, c, -1.0f, 0.0f, workspace);
}

int nsh_op_muon_step(float* w, const float* g, int64_t r, int64_t c, float lr, void* workspace) {
  return op_muon(w, g, r, c, lr * sqrtf((float)std::min(r, c)), 0.01f * lr, workspace);
}

int nsh_bench_mfma_peak(int iters, int blocks, double* tflops) {
  if (iters <= 0 || blocks <= 0 || !tflops) {
    set_error("bench_mfma_peak: bad arguments");
    return -1;
  }
  float* out = nullptr;
  NSH_CHECK(hipMalloc(&out, 256 * sizeof(float)));
  float ms = 0.f;
  const int rc = bench_mfma_peak(iters, blocks, out, &ms);
  hipFree(out);
  if (rc != 0) return -1;
  *tflops = (double)blocks * 4 * iters * 4 * 4096.0 / (ms * 1e-3) / 1e12;
  return 0;
}

int nsh_bench_copy(const float* src, float* dst, int64_t n, int reps, double* gbs) {
  if (!src || !dst || n <= 0 || n % 4 || reps <= 0 || !gbs || (((uintptr_t)src | (uintptr_t)dst) & 15)) {
    set_error("bench_copy: bad arguments");
    return -1;
  }
  float ms = 0.f;
  if (bench_copy(src, dst, n, reps, &ms) != 0) return -1;
  *gbs = 2.0 * (double)n * 4 / (ms * 1e-3) / 1e9;
  return 0;
}

int nsh_bench_rowops(const float* idx, const float* labels, int64_t M, int64_t D, int64_t V, int64_t C, int reps,
                     double* us) {
  if (!idx || !labels || M <= 0 || D <= 0 || V <= 0 || C <= 0 || reps <= 0 || !us) {
    set_error("bench_rowops: bad arguments");
    return -1;
  }
  return bench_rowops(idx, labels, M, D, V, C, reps, us);
}

int nsh_op_adamw_step(float* w, const float* g, float* m, float* v, int64_t n, int64_t t, float lr) {
  NSH_OP_REQUIRE(n >= 0 && (n == 0 || (w && g && m && v)), "adamw_step");
  const float b1t = 1.f - powf(0.9f, (float)t), b2t = 1.f - powf(0.999f, (float)t);
  if (launch_adamw(w, g, m, v, n, lr, b1t, b2t, nullptr) != 0) return -1;
  NSH_OP_DONE();
}

int nsh_op_attention_fwd(const float* Q, const float* K, const float* V, float* ctx, float* lse, int64_t S,
                         int64_t D, int64_t H) {
  NSH_OP_REQUIRE(S >= 0 && (S == 0 || (Q && K && V && ctx)), "attention_fwd");
  const void* rd[3] = {Q, K, V};
  float* pad = nullptr;  // padded copies for head sizes the tiled kernels do not take in place
  if (S > 0 && !attention_in_place(D, H, D, rd, 3) && attention_pad_floats(S, D, H, false))
    NSH_CHECK(hipMalloc(&pad, attention_pad_floats(S, D, H, false) * sizeof(float)));
  const int rc = launch_attention_fwd(Q, K, V, ctx, lse, S, D, H, D, pad, nullptr);
  const hipError_t e = hipStreamSynchronize(nullptr);
  if (pad) hipFree(pad);
  if (rc != 0) return -1;
  NSH_CHECK(e);
  return 0;
}

// workspace: delta [H*S] (rounded up to 64 floats), then dS when stored.
static size_t attn_delta_floats(int64_t S, int64_t H) { return (size_t)(ceil_div(S * H, 64) * 64); }

size_t nsh_op_attention_bwd_workspace(int64_t S, int64_t D, int64_t H, int store_ds) {
  if (S <= 0 || H <= 0 || D <= 0) return 0;
  return (attn_delta_floats(S, H) + (store_ds ? attention_bwd_ds_floats(S, D, H) : 0)) * sizeof(float);
}

int nsh_op_attention_bwd(const float* Q, const float* K, const float* V, const float* O, const float* dO,
                         const float* lse, float* dQ, float* dK, float* dV, int64_t S, int64_t D, int64_t H,
                         int store_ds, void* workspace) {
  if (!Q || !K || !V || !O || !dO || !lse || !dQ || !dK || !dV || !workspace) {
    set_error("attention_bwd: bad arguments");
    return -1;
  }
  float* delta = (float*)workspace;
  float* ds = store_ds && attention_bwd_ds_floats(S, D, H) ? delta + attn_delta_floats(S, H) : nullptr;
  const void* rd[5] = {Q, K, V, O, dO};
  float* pad = nullptr;  // padded copies for head sizes the tiled kernels do not take in place
  if (S > 0 && !attention_in_place(D, H, D, rd, 5) && attention_pad_floats(S, D, H, true))
    NSH_CHECK(hipMalloc(&pad, attention_pad_floats(S, D, H, true) * sizeof(float)));
  const int rc = launch_attention_bwd(Q, K, V, O, dO, lse, delta, dQ, dK, dV, S, D, H, D, ds, pad, nullptr);
  const hipError_t e = hipStreamSynchronize(nullptr);
  if (pad) hipFree(pad);
  if (rc != 0) return -1;
  NSH_CHECK(e);
  return 0;
}

}  // extern "C"
