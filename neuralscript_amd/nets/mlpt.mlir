// NeuralScript MLIR
ns.func @MLPT {
  ns.tensor.alloc %fc1_w : Tensor[48, 64] float32 // allocate weight [48, 64]
  ns.tensor.alloc %fc2_w : Tensor[64, 24] float32 // allocate weight [64, 24]
  ns.matmul %fc0 %x %fc1_w // x -> fc1
  ns.activation.gelu %act1 %fc0 // GELU(fc0)
  ns.matmul %fc2 %act1 %fc2_w // act1 -> fc2
  ns.return %fc2
}
ns.func @MLPT_train {
  ns.tensor.alloc %fc1_w : Tensor[48, 64] float32 // allocate weight [48, 64]
  ns.tensor.alloc %fc2_w : Tensor[64, 24] float32 // allocate weight [64, 24]
  ns.grad // gradient block (forward)
  ns.matmul %mm4 %x %fc1_w : Tensor[Bs, 64] float32 // x @ fc1_w
  ns.activation.gelu %f3 %mm4 // gelu()
  ns.matmul %mm5 %f3 %fc2_w : Tensor[Bs, 24] float32 // f3 @ fc2_w
  ns.cross_entropy %f6 %mm5 %labels // cross_entropy()
  ns.grad.loss %g7 %mm5 %labels // d(cross_entropy)/d(preds)
  ns.grad.matmul.a %g8 %g7 %fc2_w // df3 = dmm5 @ fc2_w^T
  ns.grad.matmul.w %g9 %f3 %g7 %fc2_w // dfc2_w = f3^T @ dmm5
  ns.grad.activation %g10 %g8 %mm4 // dmm4 = df3 * act'(in)
  ns.grad.matmul.a %g11 %g10 %fc1_w // dx = dmm4 @ fc1_w^T
  ns.grad.matmul.w %g12 %x %g10 %fc1_w // dfc1_w = x^T @ dmm4
  ns.opt.step %fc1_w %g12 %fc2_w %g9 // optimizer step (Muon / AdamW)
  ns.return %f6
}
