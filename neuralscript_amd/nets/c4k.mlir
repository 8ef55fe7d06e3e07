// NeuralScript MLIR
ns.func @MOE {
  ns.tensor.alloc %moe_g_w : Tensor[32, 6] float32 // allocate MoE router [32, 6]
  ns.tensor.alloc %moe_e1_w : Tensor[6, 1536] float32 // allocate MoE expert FFN-1 [6, 32 -> 48]
  ns.tensor.alloc %moe_e2_w : Tensor[6, 1536] float32 // allocate MoE expert FFN-2 [6, 48 -> 32]
  ns.layer.moe %moe0 %x %moe_g_w %moe_e1_w %moe_e2_w : Tensor[Dynamic, 32] float32 // moe(x, experts=6, ffn=48) initial=4
  ns.return %moe0
}
