// NeuralScript MLIR
ns.func @MOE {
  ns.tensor.alloc %moe_g_w : Tensor[1024, 64] float32 // allocate MoE router [1024, 64]
  ns.tensor.alloc %moe_e1_w : Tensor[64, 1048576] float32 // allocate MoE expert FFN-1 [64, 1024 -> 1024]
  ns.tensor.alloc %moe_e2_w : Tensor[64, 1048576] float32 // allocate MoE expert FFN-2 [64, 1024 -> 1024]
  ns.layer.moe %moe0 %x %moe_g_w %moe_e1_w %moe_e2_w : Tensor[Dynamic, 1024] float32 // moe(x, experts=64, ffn=1024) initial=64
  ns.return %moe0
}
