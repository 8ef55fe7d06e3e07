// NeuralScript MLIR
ns.func @SMT {
  ns.tensor.alloc %fc1_w : Tensor[8, 16] float32 // allocate weight [8, 16]
  ns.tensor.alloc %fc2_w : Tensor[16, 4] float32 // allocate weight [16, 4]
  ns.matmul %fc0 %x %fc1_w // x -> fc1
  ns.activation.softmax %f1 %fc0 // softmax()
  ns.matmul %fc2 %f1 %fc2_w // f1 -> fc2
  ns.return %fc2
}
ns.func @SMT_train {
  ns.tensor.alloc %fc1_w : Tensor[8, 16] float32 // allocate weight [8, 16]
  ns.tensor.alloc %fc2_w : Tensor[16, 4] float32 // allocate weight [16, 4]
  ns.grad // gradient block (forward)
  ns.matmul %mm3 %x %fc1_w : Tensor[B, 16] float32 // x @ fc1_w
  ns.activation.softmax %f4 %mm3 // softmax()
  ns.matmul %mm5 %f4 %fc2_w : Tensor[B, 4] float32 // f4 @ fc2_w
  ns.cross_entropy %f6 %mm5 %labels // cross_entropy()
  ns.grad.loss %g7 %mm5 %labels // d(cross_entropy)/d(preds)
  ns.grad.matmul.a %g8 %g7 %fc2_w // df4 = dmm5 @ fc2_w^T
  ns.grad.matmul.w %g9 %f4 %g7 %fc2_w // dfc2_w = f4^T @ dmm5
  ns.grad.activation %g10 %g8 %mm3 // dmm3 = df4 * act'(in)
  ns.grad.matmul.a %g11 %g10 %fc1_w // dx = dmm3 @ fc1_w^T
  ns.grad.matmul.w %g12 %x %g10 %fc1_w // dfc1_w = x^T @ dmm3
  ns.opt.step %fc1_w %g12 %fc2_w %g9 // optimizer step (Muon / AdamW)
  ns.return %f6
}
