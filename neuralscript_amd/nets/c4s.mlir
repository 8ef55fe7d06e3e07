// NeuralScript MLIR
ns.func @MOE {
  ns.tensor.alloc %moe_g_w : Tensor[64, 8] float32 // allocate MoE router [64, 8]
  ns.tensor.alloc %moe_e1_w : Tensor[8, 6144] float32 // allocate MoE expert FFN-1 [8, 64 -> 96]
  ns.tensor.alloc %moe_e2_w : Tensor[8, 6144] float32 // allocate MoE expert FFN-2 [8, 96 -> 64]
  ns.layer.moe %moe0 %x %moe_g_w %moe_e1_w %moe_e2_w : Tensor[Dynamic, 64] float32 // moe(x, experts=8, ffn=96) initial=8
  ns.return %moe0
}
