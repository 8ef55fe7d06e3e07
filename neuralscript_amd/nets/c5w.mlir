// NeuralScript MLIR
ns.func @TW {
  ns.tensor.alloc %emb_w : Tensor[128, 320] float32 // allocate embedding [128, 320]
  ns.tensor.alloc %attn_q_w : Tensor[320, 320] float32 // allocate attention weight [320, 320]
  ns.tensor.alloc %attn_k_w : Tensor[320, 320] float32 // allocate attention weight [320, 320]
  ns.tensor.alloc %attn_v_w : Tensor[320, 320] float32 // allocate attention weight [320, 320]
  ns.tensor.alloc %attn_o_w : Tensor[320, 320] float32 // allocate attention weight [320, 320]
  ns.tensor.alloc %mlp1_w : Tensor[320, 256] float32 // allocate weight [320, 256]
  ns.tensor.alloc %mlp2_w : Tensor[256, 320] float32 // allocate weight [256, 320]
  ns.tensor.alloc %fc_w : Tensor[320, 128] float32 // allocate weight [320, 128]
  ns.layer.embedding %emb0 %emb_w %x : Tensor[Dynamic, 320] float32 // embedding(x, emb_w)
  ns.layer.attention %attn1 %emb0 %attn_q_w %attn_k_w %attn_v_w %attn_o_w : Tensor[Dynamic, 320] float32 // attention(emb0, heads=2)
  ns.layernorm %ln2 %attn1 : Tensor[T, 320] float32 // layernorm(attn1)
  ns.matmul %fc3 %ln2 %mlp1_w // ln2 -> mlp1
  ns.activation.relu %act4 %fc3 // ReLU(fc3)
  ns.matmul %fc5 %act4 %mlp2_w // act4 -> mlp2
  ns.matmul %fc6 %fc5 %fc_w // fc5 -> fc
  ns.return %fc6
}
ns.func @TW_train {
  ns.tensor.alloc %emb_w : Tensor[128, 320] float32 // allocate embedding [128, 320]
  ns.tensor.alloc %attn_q_w : Tensor[320, 320] float32 // allocate attention weight [320, 320]
  ns.tensor.alloc %attn_k_w : Tensor[320, 320] float32 // allocate attention weight [320, 320]
  ns.tensor.alloc %attn_v_w : Tensor[320, 320] float32 // allocate attention weight [320, 320]
  ns.tensor.alloc %attn_o_w : Tensor[320, 320] float32 // allocate attention weight [320, 320]
  ns.tensor.alloc %mlp1_w : Tensor[320, 256] float32 // allocate weight [320, 256]
  ns.tensor.alloc %mlp2_w : Tensor[256, 320] float32 // allocate weight [256, 320]
  ns.tensor.alloc %fc_w : Tensor[320, 128] float32 // allocate weight [320, 128]
  ns.grad // gradient block (forward)
  ns.layer.embedding %emb7 %emb_w %x : Tensor[Dynamic, 320] float32 // embedding(x, emb_w)
  ns.layer.attention %attn8 %emb7 %attn_q_w %attn_k_w %attn_v_w %attn_o_w : Tensor[Dynamic, 320] float32 // attention(emb7, heads=2)
  ns.layernorm %ln9 %attn8 : Tensor[T, 320] float32 // layernorm(attn8)
  ns.matmul %mm11 %ln9 %mlp1_w : Tensor[T, 256] float32 // ln9 @ mlp1_w
  ns.activation.relu %f10 %mm11 // relu()
  ns.matmul %mm12 %f10 %mlp2_w : Tensor[T, 320] float32 // f10 @ mlp2_w
  ns.matmul %mm13 %mm12 %fc_w : Tensor[T, 128] float32 // mm12 @ fc_w
  ns.cross_entropy %f14 %mm13 %labels // cross_entropy()
  ns.grad.loss %g15 %mm13 %labels // d(cross_entropy)/d(preds)
  ns.grad.matmul.a %g16 %g15 %fc_w // dmm12 = dmm13 @ fc_w^T
  ns.grad.matmul.w %g17 %mm12 %g15 %fc_w // dfc_w = mm12^T @ dmm13
  ns.grad.matmul.a %g18 %g16 %mlp2_w // df10 = dmm12 @ mlp2_w^T
  ns.grad.matmul.w %g19 %f10 %g16 %mlp2_w // dmlp2_w = f10^T @ dmm12
  ns.grad.activation %g20 %g18 %mm11 // dmm11 = df10 * act'(in)
  ns.grad.matmul.a %g21 %g20 %mlp1_w // dln9 = dmm11 @ mlp1_w^T
  ns.grad.matmul.w %g22 %ln9 %g20 %mlp1_w // dmlp1_w = ln9^T @ dmm11
  ns.grad.layernorm %g23 %g21 %attn8 // dattn8 = layernorm_grad(dln9, attn8)
  ns.grad.attention.x %g24 %g23 %emb7 %attn_q_w %attn_k_w %attn_v_w %attn_o_w // dx(attention)
  ns.grad.attention.wq %g25 %g23 %emb7 %attn_q_w %attn_k_w %attn_v_w %attn_o_w // 
  ns.grad.attention.wk %g26 %g23 %emb7 %attn_q_w %attn_k_w %attn_v_w %attn_o_w // 
  ns.grad.attention.wv %g27 %g23 %emb7 %attn_q_w %attn_k_w %attn_v_w %attn_o_w // 
  ns.grad.attention.wo %g28 %g23 %emb7 %attn_q_w %attn_k_w %attn_v_w %attn_o_w // 
  ns.grad.embedding.w %g29 %g24 %x %emb_w // demb_w = scatter_add(demb7)
  ns.opt.step %emb_w %g29 %attn_q_w %g25 %attn_k_w %g26 %attn_v_w %g27 %attn_o_w %g28 %mlp1_w %g22 %mlp2_w %g19 %fc_w %g17 // optimizer step (Muon / AdamW)
  ns.return %f14
}
