// NeuralScript MLIR
ns.func @DRP {
  ns.tensor.alloc %fc1_w : Tensor[8, 16] float32 // allocate weight [8, 16]
  ns.tensor.alloc %fc2_w : Tensor[16, 16] float32 // allocate weight [16, 16]
  ns.tensor.alloc %fc3_w : Tensor[16, 4] float32 // allocate weight [16, 4]
  ns.matmul %fc0 %x %fc1_w // x -> fc1
  ns.activation.relu %act1 %fc0 // ReLU(fc0)
  ns.dropout %fc2 %act1 // dropout(act1, p=0.250000) rate=0.25
  ns.matmul %fc3 %fc2 %fc2_w // fc2 -> fc2
  ns.activation.gelu %act4 %fc3 // GELU(fc3)
  ns.dropout %fc5 %act4 // dropout(act4, p=0.100000) rate=0.10000000000000001
  ns.matmul %fc6 %fc5 %fc3_w // fc5 -> fc3
  ns.return %fc6
}
ns.func @DRP_train {
  ns.tensor.alloc %fc1_w : Tensor[8, 16] float32 // allocate weight [8, 16]
  ns.tensor.alloc %fc2_w : Tensor[16, 16] float32 // allocate weight [16, 16]
  ns.tensor.alloc %fc3_w : Tensor[16, 4] float32 // allocate weight [16, 4]
  ns.grad // gradient block (forward)
  ns.matmul %fc7 %x %fc1_w // x -> fc1
  ns.activation.relu %act8 %fc7 // ReLU(fc7)
  ns.dropout %fc9 %act8 // dropout(act8, p=0.250000) rate=0.25
  ns.matmul %fc10 %fc9 %fc2_w // fc9 -> fc2
  ns.activation.gelu %act11 %fc10 // GELU(fc10)
  ns.dropout %fc12 %act11 // dropout(act11, p=0.100000) rate=0.10000000000000001
  ns.matmul %fc13 %fc12 %fc3_w // fc12 -> fc3
  ns.cross_entropy %f14 %fc13 %labels // cross_entropy()
  ns.grad.loss %g15 %fc13 %labels // d(cross_entropy)/d(preds)
  ns.grad.matmul.a %g16 %g15 %fc3_w // dfc12 = dfc13 @ fc3_w^T
  ns.grad.matmul.w %g17 %fc12 %g15 %fc3_w // dfc3_w = fc12^T @ dfc13
  ns.grad.activation %g18 %g16 %fc12 // dact11 = dfc12 * dropout_mask
  ns.grad.activation %g19 %g18 %fc10 // dfc10 = dact11 * act'(in)
  ns.grad.matmul.a %g20 %g19 %fc2_w // dfc9 = dfc10 @ fc2_w^T
  ns.grad.matmul.w %g21 %fc9 %g19 %fc2_w // dfc2_w = fc9^T @ dfc10
  ns.grad.activation %g22 %g20 %fc9 // dact8 = dfc9 * dropout_mask
  ns.grad.activation %g23 %g22 %fc7 // dfc7 = dact8 * act'(in)
  ns.grad.matmul.a %g24 %g23 %fc1_w // dx = dfc7 @ fc1_w^T
  ns.grad.matmul.w %g25 %x %g23 %fc1_w // dfc1_w = x^T @ dfc7
  ns.opt.step %fc1_w %g25 %fc2_w %g21 %fc3_w %g17 // optimizer step (Muon / AdamW)
  ns.return %f14
}
