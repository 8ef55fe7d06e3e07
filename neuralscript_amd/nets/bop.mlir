// NeuralScript MLIR
ns.func @BOP {
  ns.tensor.alloc %fc1_w : Tensor[8, 8] float32 // allocate weight [8, 8]
  ns.tensor.alloc %fc2_w : Tensor[8, 8] float32 // allocate weight [8, 8]
  ns.tensor.alloc %B2 : Tensor[1, 8] float32 // allocate Tensor[1, 8] float32
  ns.matmul %fc0 %x %fc1_w // x -> fc1
  ns.activation.softmax %f1 %fc0 // softmax()
  ns.subview_binop %e2 %f1 %B2 //  op=
  ns.subview_binop %e3 %e2 %x //  op=
  ns.matmul %fc4 %e3 %fc2_w // e3 -> fc2
  ns.activation.tanh %act5 %fc4 // Tanh(fc4)
  ns.subview_binop %e6 %act5 %act5 //  op=
  ns.constant %c7 // constant 1.5 value=1.5
  ns.subview_binop %e8 %e6 %c7 //  op=
  ns.layernorm %ln9 %act5 : Tensor[1, 8] float32 // layernorm(act5)
  ns.subview_binop %e10 %ln9 %B2 //  op=
  ns.activation.softmax %f11 %ln9 // softmax()
  ns.subview_binop %e12 %f11 %e8 //  op=
  ns.return %e12
}
