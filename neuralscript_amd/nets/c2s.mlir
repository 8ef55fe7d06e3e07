// NeuralScript MLIR
ns.func @MLP {
  ns.tensor.alloc %fc1_w : Tensor[96, 160] float32 // allocate weight [96, 160]
  ns.tensor.alloc %fc2_w : Tensor[160, 128] float32 // allocate weight [160, 128]
  ns.tensor.alloc %fc3_w : Tensor[128, 80] float32 // allocate weight [128, 80]
  ns.matmul %fc0 %x %fc1_w // x -> fc1
  ns.activation.gelu %act1 %fc0 // GELU(fc0)
  ns.matmul %fc2 %act1 %fc2_w // act1 -> fc2
  ns.activation.gelu %act3 %fc2 // GELU(fc2)
  ns.matmul %fc4 %act3 %fc3_w // act3 -> fc3
  ns.return %fc4
}
