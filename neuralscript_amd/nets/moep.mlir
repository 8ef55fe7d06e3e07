// NeuralScript MLIR
ns.func @MoEP {
  ns.tensor.alloc %emb_w : Tensor[8192, 1024] float32 // allocate embedding [8192, 1024]
  ns.tensor.alloc %moe_g_w : Tensor[1024, 64] float32 // allocate MoE router [1024, 64]
  ns.tensor.alloc %moe_e1_w : Tensor[64, 1048576] float32 // allocate MoE expert FFN-1 [64, 1024 -> 1024]
  ns.tensor.alloc %moe_e2_w : Tensor[64, 1048576] float32 // allocate MoE expert FFN-2 [64, 1024 -> 1024]
  ns.tensor.alloc %fc_w : Tensor[1024, 16] float32 // allocate weight [1024, 16]
  ns.layer.embedding %emb0 %emb_w %x : Tensor[Dynamic, 1024] float32 // embedding(x, emb_w)
  ns.layer.moe %moe1 %emb0 %moe_g_w %moe_e1_w %moe_e2_w : Tensor[Dynamic, 1024] float32 // moe(emb0, experts=64, ffn=1024) initial=64
  ns.matmul %fc2 %moe1 %fc_w // moe1 -> fc
  ns.return %fc2
}
ns.func @MoEP_train {
  ns.tensor.alloc %emb_w : Tensor[8192, 1024] float32 // allocate embedding [8192, 1024]
  ns.tensor.alloc %moe_g_w : Tensor[1024, 64] float32 // allocate MoE router [1024, 64]
  ns.tensor.alloc %moe_e1_w : Tensor[64, 1048576] float32 // allocate MoE expert FFN-1 [64, 1024 -> 1024]
  ns.tensor.alloc %moe_e2_w : Tensor[64, 1048576] float32 // allocate MoE expert FFN-2 [64, 1024 -> 1024]
  ns.tensor.alloc %fc_w : Tensor[1024, 16] float32 // allocate weight [1024, 16]
  ns.grad // gradient block (forward)
  ns.layer.embedding %emb3 %emb_w %x : Tensor[Dynamic, 1024] float32 // embedding(x, emb_w)
  ns.layer.moe %moe4 %emb3 %moe_g_w %moe_e1_w %moe_e2_w : Tensor[Dynamic, 1024] float32 // moe(emb3, experts=64, ffn=1024) initial=64
  ns.matmul %mm5 %moe4 %fc_w : Tensor[B, 16] float32 // moe4 @ fc_w
  ns.cross_entropy %f6 %mm5 %labels // cross_entropy()
  ns.grad.loss %g7 %mm5 %labels // d(cross_entropy)/d(preds)
  ns.grad.matmul.a %g8 %g7 %fc_w // dmoe4 = dmm5 @ fc_w^T
  ns.grad.matmul.w %g9 %moe4 %g7 %fc_w // dfc_w = moe4^T @ dmm5
  ns.grad.moe.x %g10 %g8 %emb3 %moe_g_w %moe_e1_w %moe_e2_w // dx(moe)
  ns.grad.moe.wg %g11 %g8 %emb3 %moe_g_w %moe_e1_w %moe_e2_w // dWg(moe)
  ns.grad.moe.we1 %g12 %g8 %emb3 %moe_g_w %moe_e1_w %moe_e2_w // dWe1(moe)
  ns.grad.moe.we2 %g13 %g8 %emb3 %moe_g_w %moe_e1_w %moe_e2_w // dWe2(moe)
  ns.grad.embedding.w %g14 %g10 %x %emb_w // demb_w = scatter_add(demb3)
  ns.opt.step %emb_w %g14 %moe_g_w %g11 %moe_e1_w %g12 %moe_e2_w %g13 %fc_w %g9 // optimizer step (Muon / AdamW)
  ns.return %f6
}
