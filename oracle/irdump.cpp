// irdump: prints the reference compiler's IR for a .ns program in the exact
// text format of `nsc --mlir` (MLIRCompiler::dump, mlir_compiler.cpp:949-1025),
// with the instruction attributes that dump leaves out appended to each
// instruction's comment as key=value tokens:
//
//   ns.subview_binop   op=+|-|*|/            (MLIRInstr::attribute)
//   ns.constant        value=<literal>
//   ns.concat          axis=<0|1>
//   ns.reshape         shape=<r>:<c>
//   ns.slice           axis=<a> start=<s> stop=<e>
//   ns.index/scatter   axis=<a> idx=<i0,i1,...>   (int_attr, ints_attr)
//   ns.dropout         rate=<p>              (float_attr, 17 significant digits)
//   ns.layer.moe       initial=<K0>          (ints_attr[0], mlir_compiler.cpp:896)
//
// libnship's plan parser reads these keys.  Test/build infrastructure only:
// linked against the reference compiler's objects by oracle/Makefile.
#include "ns/lexer/lexer.hpp"
#include "ns/mlir/mlir_compiler.hpp"
#include "ns/parser/parser.hpp"
#include "ns/typechecker/shape_checker.hpp"

#include <fstream>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

namespace {

std::string attrs_of(const ns::MLIRInstr& in) {
  using ns::MLIROp;
  std::ostringstream o;
  auto ints = [&]() {
    std::string s;
    for (size_t k = 0; k < in.ints_attr.size(); k++) s += (k ? "," : "") + std::to_string(in.ints_attr[k]);
    return s;
  };
  switch (in.op) {
    case MLIROp::ELEMENTWISE_BINOP: o << "op=" << in.attribute; break;
    case MLIROp::CONSTANT: o << "value=" << in.attribute; break;
    case MLIROp::CONCAT: o << "axis=" << (in.attribute.empty() ? "1" : in.attribute); break;
    case MLIROp::RESHAPE:
      if (!in.attribute.empty()) o << "shape=" << in.attribute;
      break;
    case MLIROp::SLICE: {
      int axis = 1, s = 0, e = 0;
      char c;
      std::istringstream is(in.attribute);
      is >> axis >> c >> s >> c >> e;
      o << "axis=" << axis << " start=" << s << " stop=" << e;
      break;
    }
    case MLIROp::INDEX: case MLIROp::SCATTER: o << "axis=" << in.int_attr << " idx=" << ints(); break;
    case MLIROp::DROPOUT: {
      // exact value: the emitted code prints it with std::to_string
      std::ostringstream r;
      r.precision(17);
      r << in.float_attr;
      o << "rate=" << r.str();
      break;
    }
    case MLIROp::LAYER_MOE:
      if (!in.ints_attr.empty()) o << "initial=" << in.ints_attr[0];
      break;
    default: break;
  }
  return o.str();
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 2) {
    std::cerr << "usage: irdump <file.ns>\n";
    return 1;
  }
  std::ifstream f(argv[1]);
  if (!f) {
    std::cerr << "cannot open " << argv[1] << "\n";
    return 1;
  }
  std::ostringstream src;
  src << f.rdbuf();
  try {
    ns::Lexer lexer(src.str());
    auto tokens = lexer.tokenize();
    ns::Parser parser(tokens);
    ns::Program program = parser.parse_program();
    ns::ShapeChecker checker;
    if (!checker.check(program)) {
      for (auto& e : checker.errors()) std::cerr << e.line << ":" << e.column << "  " << e.message << "\n";
      return 1;
    }
    ns::MLIRCompiler mlir;
    auto module = mlir.compile(program);
    // The dump prints, per function: a header line, one line per
    // instruction in order, an optional return line and a closing brace.
    std::istringstream text(mlir.dump(module));
    std::string line;
    std::getline(text, line);  // "// NeuralScript MLIR"
    std::cout << line << "\n";
    for (auto& fn : module.functions) {
      std::getline(text, line);  // ns.func @name {
      std::cout << line << "\n";
      for (auto& in : fn.instructions) {
        std::getline(text, line);
        const std::string a = attrs_of(in);
        std::cout << line << (a.empty() ? "" : " " + a) << "\n";
      }
      while (std::getline(text, line)) {
        std::cout << line << "\n";
        if (line == "}") break;
      }
    }
  } catch (const std::exception& e) {
    std::cerr << "error: " << e.what() << "\n";
    return 1;
  }
  return 0;
}
