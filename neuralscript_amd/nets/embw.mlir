// NeuralScript MLIR
ns.func @EW {
  ns.tensor.alloc %emb_w : Tensor[4096, 64] float32 // allocate embedding [4096, 64]
  ns.tensor.alloc %fc_w : Tensor[64, 128] float32 // allocate weight [64, 128]
  ns.layer.embedding %emb0 %emb_w %x : Tensor[Dynamic, 64] float32 // embedding(x, emb_w)
  ns.matmul %fc1 %emb0 %fc_w // emb0 -> fc
  ns.return %fc1
}
ns.func @EW_train {
  ns.tensor.alloc %emb_w : Tensor[4096, 64] float32 // allocate embedding [4096, 64]
  ns.tensor.alloc %fc_w : Tensor[64, 128] float32 // allocate weight [64, 128]
  ns.grad // gradient block (forward)
  ns.layer.embedding %emb2 %emb_w %x : Tensor[Dynamic, 64] float32 // embedding(x, emb_w)
  ns.matmul %mm3 %emb2 %fc_w : Tensor[T, 128] float32 // emb2 @ fc_w
  ns.cross_entropy %f4 %mm3 %labels // cross_entropy()
  ns.grad.loss %g5 %mm3 %labels // d(cross_entropy)/d(preds)
  ns.grad.matmul.a %g6 %g5 %fc_w // demb2 = dmm3 @ fc_w^T
  ns.grad.matmul.w %g7 %emb2 %g5 %fc_w // dfc_w = emb2^T @ dmm3
  ns.grad.embedding.w %g8 %g6 %x %emb_w // demb_w = scatter_add(demb2)
  ns.opt.step %emb_w %g8 %fc_w %g7 // optimizer step (Muon / AdamW)
  ns.return %f4
}
