// NeuralScript MLIR
ns.func @MLP {
  ns.tensor.alloc %fc1_w : Tensor[64, 256] float32 // allocate weight [64, 256]
  ns.tensor.alloc %fc2_w : Tensor[256, 256] float32 // allocate weight [256, 256]
  ns.tensor.alloc %fc3_w : Tensor[256, 10] float32 // allocate weight [256, 10]
  ns.matmul %fc0 %x %fc1_w // x -> fc1
  ns.activation.relu %act1 %fc0 // ReLU(fc0)
  ns.matmul %fc2 %act1 %fc2_w // act1 -> fc2
  ns.activation.relu %act3 %fc2 // ReLU(fc2)
  ns.matmul %fc4 %act3 %fc3_w // act3 -> fc3
  ns.return %fc4
}
