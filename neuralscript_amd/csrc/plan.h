// Network plan: the instruction list of `nsc --mlir` (printer at
// /root/reference/src/mlir/mlir_compiler.cpp:949-1025), resolved into value
// ids, weight offsets and per-op attributes.  Attributes that printer drops
// arrive as key=value tokens in the instruction comment (initial=, op=,
// value=, axis=, start=, stop=, idx=, rate=).  Pure host code.
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "ns_runtime.h"

namespace nship {

enum class Op {
  Alloc, Marker, Matmul, Act, Dropout, LayerNorm, Embedding, Attention, Moe, CrossEntropy,
  LossGrad, MatmulGradA, MatmulGradW, ActGrad, LayerNormGrad, EmbeddingGradW,
  AttnGradX, AttnGradWq, AttnGradWk, AttnGradWv, AttnGradWo,
  MoeGradX, MoeGradWg, MoeGradWe1, MoeGradWe2, OptStep,
  // forward-only ops (codegen.cpp:2007-2018, 2027-2033, 2079-2203)
  Binop, Softmax, Constant, Transpose, Concat, Reshape, Slice, Index, Scatter
};

struct Instr {
  Op op = Op::Marker;
  int res = -1;               // value id of the result (-1: none)
  std::vector<int> in;        // operand value ids
  int act = 0;                // Act / ActGrad: activation code; Matmul: fused epilogue
  int64_t rt_cols = -1;       // column count from the printed result type
  int heads = 1;              // Attention / AttnGrad*
  bool fused_away = false;    // Act folded into the preceding Matmul
  // Epilogue absorbed into a GEMM group by the reference's fusion pass
  // (fusion.cpp:52-175): binops become the identity, softmax / layernorm
  // run over rows of the GEMM's N (codegen.cpp:2052-2076).
  bool in_group = false;
  int64_t group_n = 0;
  int64_t k = 0, n = 0;       // Matmul: static K, N of the B operand
  int binop = 0;              // Binop: 0 +, 1 -, 2 *, 3 /
  int axis = 1;               // Concat / Slice / Index / Scatter
  int64_t start = 0, stop = 0;  // Slice
  std::vector<int64_t> idx;   // Index / Scatter
  float value = 0.f;          // Constant
  double rate = 0.0;          // Dropout: float_attr; ActGrad of a dropout: that dropout's
  bool dropout = false;       // ActGrad: the gradient of a dropout (dIn = dOut * its mask)
  // OptStep with `optimizer=adamw` in its comment: every weight takes AdamW.
  // A build knob of this backend, not something the reference emits (its
  // rule is by shape, codegen.cpp:3097).
  bool adamw_only = false;
};

struct Value {
  std::string name;
  bool weight = false;
  int64_t rows = -1, cols = -1;  // weights: static shape
  size_t offset = 0;             // weights: float offset in the blob
};

struct Func {
  std::string name;
  std::vector<Instr> ins;
  int ret = -1;
  bool train = false;
  int x = -1;  // runtime data input
  int y = -1;  // labels (training)
  std::vector<int64_t> width;  // propagated column count per value id (-1 unknown)
  // the emitted code's static shape table (codegen.cpp:1170-1224):
  // per value id, rows / cols from result types and weight shapes, -1 = dynamic
  std::vector<int64_t> srows, scols;
};

struct MoeInfo {
  bool present = false;
  int64_t D = 0, E = 0, H = 0, K0 = 0;
  int g = -1, e1 = -1, e2 = -1;  // weight value ids
};

// The runtime wrapper's learning-rate multiplier (optim_params.hpp:36-62),
// compiled into the reference's driver from optim::kLRSchedule and carried
// here by the IR line `// ns.lr_schedule <kind> warmup=W total=T min=F`
// (kind constant | cosine_warmup; absent: constant, the reference default).
struct LrSchedule {
  int kind = 0;  // 0 constant, 1 linear warmup then cosine decay
  int64_t warmup = 100, total = 10000;
  float min_factor = 0.05f;
};
// Multiplier at wrapper step `step` (codegen.cpp:23-39 / optim_params.hpp:54-62).
float lr_scale(const LrSchedule& s, int64_t step);

struct Plan {
  LrSchedule lr;
  std::vector<Value> vals;
  std::map<std::string, int> index;
  std::vector<int> weights;  // value ids in TENSOR_ALLOC order
  Func fwd, trn;
  bool has_train = false;
  size_t total = 0;
  int64_t in_cols = 1, out_cols = 1;
  MoeInfo moe;
  std::vector<std::string> wnames;
  std::vector<ns_weight_desc> desc;
  ns_weight_layout layout{0, nullptr};
};

// Parses the IR text.  On failure returns nullptr and sets *err.
Plan* parse_plan(const char* text, std::string* err);

}  // namespace nship
