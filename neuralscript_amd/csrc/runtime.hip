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

#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <random>
#include <string>
#include <vector>

#include "common.h"
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
};

struct ns_model {
  const Plan* plan = nullptr;
  hipStream_t stream = nullptr;
  float* d_w = nullptr;
  std::vector<float> h_w;
  bool host_stale = false;  // device blob newer than h_w
  std::vector<uint8_t> moe_active;
  size_t moe_count = 0;
  uint8_t* d_active = nullptr;
  std::mt19937 rng{0x9E3779B9u};  // codegen.cpp:2421
  int64_t lr_step = 0;
  int64_t moe_last_m = 0;         // tokens routed by the last MoE forward
  std::vector<Buf> arena;         // per value id
  std::map<std::string, Buf> scratch;
  // profiling
  bool prof = false;
  std::vector<ProfEntry> pending;
  std::vector<hipEvent_t> event_pool;
  std::map<std::string, std::pair<long, double>> prof_acc;
};

namespace nship {
namespace {

int ensure(Buf& b, size_t n) {
  if (n <= b.cap) return 0;
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
    if (m->prof && (a = take_event(m))) hipEventRecord(a, m->stream);
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
};

float* scratch(ns_model* m, const std::string& key, size_t n) {
  Buf& b = m->scratch[key];
  if (ensure(b, n) != 0) return nullptr;
  return b.p;
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

float* out_buf(ns_model* m, Frame& fr, int id, size_t n) {
  if (ensure(m->arena[id], n) != 0) return nullptr;
  fr.numel[id] = n;
  fr.ptr[id] = m->arena[id].p;
  return fr.ptr[id];
}

#define NSH_OUT(var, id, n)                          \
  float* var = out_buf(m, fr, (id), (n));            \
  if (!var) return -1

// Forward instructions (shared by inference and the training forward).
int exec_forward_op(ns_model* m, const Func& F, const Instr& I, Frame& fr, bool train) {
  const Plan& P = *m->plan;
  hipStream_t s = m->stream;
  switch (I.op) {
    case Op::Matmul: {
      const Value& B = P.vals[I.in[1]];
      const int64_t K = B.rows, N = B.cols;
      const int64_t M = (int64_t)(fr.numel[I.in[0]] / (size_t)K);
      NSH_OUT(C, I.res, (size_t)(M * N));
      Prof p(m, I.act ? "gemm_act" : "gemm");
      return launch_gemm(fr.ptr[I.in[0]], fr.ptr[I.in[1]], C, M, N, K, K, N, N, false, false, I.act, s);
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
          if (launch_gemm_ex(g, false, false, 3, s) != 0) return -1;
        } else {
          for (int j = 0; j < 3; j++) {
            g.B = fr.ptr[I.in[1 + j]];
            g.C = sv.qkv + j * BS * D;
            if (launch_gemm_ex(g, false, false, 1, s) != 0) return -1;
          }
        }
      }
      {
        Prof p(m, "attention_fwd");
        if (launch_attention_fwd(sv.qkv, sv.qkv + BS * D, sv.qkv + 2 * BS * D, sv.ctx, train ? sv.lse : nullptr, BS, D,
                                 H, D, s) != 0)
          return -1;
      }
      Prof p(m, "gemm");
      return launch_gemm(sv.ctx, fr.ptr[I.in[4]], out, BS, D, D, D, D, D, false, false, 0, s);
    }
    case Op::Moe: {
      const MoeInfo& q = P.moe;
      const int64_t M = (int64_t)(fr.numel[I.in[0]] / (size_t)q.D);
      NSH_OUT(out, I.res, (size_t)(M * q.D));
      MoeWork w;
      if (moe_work(m, M, &w) != 0) return -1;
      Prof p(m, "moe");
      if (launch_moe_route(fr.ptr[I.in[0]], fr.ptr[I.in[1]], m->d_active, w, M, q.D, q.E, s) != 0) return -1;
      m->moe_last_m = M;
      return launch_moe_experts(fr.ptr[I.in[0]], fr.ptr[I.in[2]], fr.ptr[I.in[3]], w, out, M, q.D, q.H, q.E, s);
    }
    case Op::Dropout:
      if (train) {
        set_error("dropout in training is not supported");
        return -1;
      }
      fr.numel[I.res] = fr.numel[I.in[0]];
      fr.ptr[I.res] = fr.ptr[I.in[0]];
      return 0;
    default:
      break;
  }
  (void)F;
  set_error("instruction not supported by this build of libnship");
  return -1;
}

int run_forward(ns_model* m, const float* d_x, size_t n_in, float** d_out, size_t* n_out) {
  const Plan& P = *m->plan;
  const Func& F = P.fwd;
  Frame fr;
  bind_weights(m, fr);
  fr.numel[F.x] = n_in;
  fr.ptr[F.x] = const_cast<float*>(d_x);
  for (const Instr& I : F.ins) {
    if (I.fused_away || I.op == Op::Marker) continue;
    if (exec_forward_op(m, F, I, fr, false) != 0) return -1;
  }
  if (F.ret < 0) {
    set_error("forward function has no return value");
    return -1;
  }
  *d_out = fr.ptr[F.ret];
  *n_out = fr.numel[F.ret];
  return 0;
}

int host_sync_weights(const ns_model* m) {
  if (!m->host_stale) return 0;
  ns_model* mm = const_cast<ns_model*>(m);
  NSH_CHECK(hipStreamSynchronize(mm->stream));
  NSH_CHECK(hipMemcpy(mm->h_w.data(), mm->d_w, mm->h_w.size() * sizeof(float), hipMemcpyDeviceToHost));
  mm->host_stale = false;
  return 0;
}

int device_sync_weights(ns_model* m) {
  NSH_CHECK(hipMemcpy(m->d_w, m->h_w.data(), m->h_w.size() * sizeof(float), hipMemcpyHostToDevice));
  if (m->d_active && !m->moe_active.empty())
    NSH_CHECK(hipMemcpy(m->d_active, m->moe_active.data(), m->moe_active.size(), hipMemcpyHostToDevice));
  return 0;
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

int nsh_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  NSH_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return 0;
}

int nsh_memcpy_d2h(void* dst, const void* src, size_t bytes) {
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

void nsh_plan_free(nsh_plan* p) { delete p; }
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
  for (auto& b : m->arena) if (b.p) hipFree(b.p);
  for (auto& kv : m->scratch) if (kv.second.p) hipFree(kv.second.p);
  for (auto& e : m->pending) { hipEventDestroy(e.a); hipEventDestroy(e.b); }
  for (auto e : m->event_pool) hipEventDestroy(e);
  if (m->d_w) hipFree(m->d_w);
  if (m->d_active) hipFree(m->d_active);
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
  if (run_forward(m, d_input, input_numel, &res, &n) != 0) return -1;
  if (n) NSH_CHECK(hipMemcpyAsync(d_output, res, n * sizeof(float), hipMemcpyDeviceToDevice, m->stream));
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
  NSH_CHECK(hipMemcpyAsync(xb.p, input, input_numel * sizeof(float), hipMemcpyHostToDevice, m->stream));
  float* res = nullptr;
  size_t n = 0;
  if (run_forward(m, xb.p, input_numel, &res, &n) != 0) return -1;
  if (n) NSH_CHECK(hipMemcpyAsync(output, res, n * sizeof(float), hipMemcpyDeviceToHost, m->stream));
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
  }
  device_sync_weights(m);
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
  device_sync_weights(m);
  return m->moe_count;
}

size_t nsh_expert_kill(ns_model* m, int k) {
  if (!m) return 0;
  const MoeInfo& q = m->plan->moe;
  if (!q.present || k < 0 || k >= (int)q.E || !m->moe_active[(size_t)k]) return m->moe_count;
  m->moe_active[(size_t)k] = 0;
  m->moe_count--;
  device_sync_weights(m);
  return m->moe_count;
}

int nsh_train_step(ns_model* m, const float* input, const float* labels, size_t input_numel,
                   float* loss_out, float lr) {
  (void)m; (void)input; (void)labels; (void)input_numel; (void)loss_out; (void)lr;
  set_error("training is not available in this build");
  return -1;
}

int nsh_objective_loss(ns_model* m, const float* input, const float* labels, size_t input_numel,
                       float* loss_out) {
  (void)m; (void)input; (void)labels; (void)input_numel; (void)loss_out;
  set_error("training is not available in this build");
  return -1;
}

// ---- profiling ---------------------------------------------------------------
int nsh_profile_enable(ns_model* m, int on) {
  if (!m) return -1;
  if (sync(m) != 0) return -1;
  m->prof = on != 0;
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

#define NSH_OP_DONE()                             \
  do {                                            \
    NSH_CHECK(hipStreamSynchronize(nullptr));     \
    return 0;                                     \
  } while (0)

int nsh_op_embedding(const float* W, const float* idx, float* out, int64_t n, int64_t V, int64_t D) {
  if (launch_embedding(W, idx, out, n, V, D, nullptr) != 0) return -1;
  NSH_OP_DONE();
}

int nsh_op_layernorm(const float* x, float* y, int64_t rows, int64_t last) {
  if (last <= 0 || launch_layernorm(x, y, rows, last, nullptr) != 0) return -1;
  NSH_OP_DONE();
}

int nsh_op_layernorm_grad(const float* dout, const float* x, float* dx, int64_t rows, int64_t last) {
  if (last <= 0 || launch_layernorm_grad(dout, x, dx, rows, last, nullptr) != 0) return -1;
  NSH_OP_DONE();
}

int nsh_op_softmax_xent(const float* logits, const float* labels, float* grad, float* row_loss, float* loss,
                        int64_t rows, int64_t C) {
  if (launch_softmax_xent(logits, labels, grad, row_loss, loss, rows, C, grad != nullptr, nullptr) != 0) return -1;
  NSH_OP_DONE();
}

int nsh_op_act_grad(const float* din, const float* pre, float* dout, int64_t n, int act) {
  if (launch_act_grad(din, pre, dout, n, act, nullptr) != 0) return -1;
  NSH_OP_DONE();
}

size_t nsh_op_embedding_grad_workspace(int64_t n, int64_t V) { return embedding_grad_workspace(n, V) * sizeof(int); }

int nsh_op_embedding_grad(const float* dout, const float* idx, float* dW, int64_t n, int64_t V, int64_t D,
                          void* workspace) {
  if (!workspace || launch_embedding_grad(dout, idx, dW, n, V, D, (int*)workspace, nullptr) != 0) return -1;
  NSH_OP_DONE();
}

int nsh_op_attention_fwd(const float* Q, const float* K, const float* V, float* ctx, float* lse, int64_t S,
                         int64_t D, int64_t H) {
  if (launch_attention_fwd(Q, K, V, ctx, lse, S, D, H, D, nullptr) != 0) return -1;
  NSH_OP_DONE();
}

}  // extern "C"
