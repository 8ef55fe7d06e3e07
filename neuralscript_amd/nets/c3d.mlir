// NeuralScript MLIR
ns.func @EAL8 {
  ns.tensor.alloc %emb_w : Tensor[32000, 1024] float32 // allocate embedding [32000, 1024]
  ns.tensor.alloc %attn_q_w : Tensor[1024, 1024] float32 // allocate attention weight [1024, 1024]
  ns.tensor.alloc %attn_k_w : Tensor[1024, 1024] float32 // allocate attention weight [1024, 1024]
  ns.tensor.alloc %attn_v_w : Tensor[1024, 1024] float32 // allocate attention weight [1024, 1024]
  ns.tensor.alloc %attn_o_w : Tensor[1024, 1024] float32 // allocate attention weight [1024, 1024]
  ns.layer.embedding %emb0 %emb_w %x : Tensor[Dynamic, 1024] float32 // embedding(x, emb_w)
  ns.layer.attention %attn1 %emb0 %attn_q_w %attn_k_w %attn_v_w %attn_o_w : Tensor[Dynamic, 1024] float32 // attention(emb0, heads=8)
  ns.layernorm %ln2 %attn1 : Tensor[T, 1024] float32 // layernorm(attn1)
  ns.return %ln2
}
