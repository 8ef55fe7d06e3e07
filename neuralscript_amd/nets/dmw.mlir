// NeuralScript MLIR
ns.func @DMW {
  ns.tensor.alloc %A : Tensor[3, 4] float32 // allocate Tensor[3, 4] float32
  ns.tensor.alloc %P : Tensor[4, 6] float32 // allocate Tensor[4, 6] float32
  ns.tensor.alloc %U : Tensor[2, 4] float32 // allocate Tensor[2, 4] float32
  ns.matmul %mm0 %x %P : Tensor[B, 6] float32 // x @ P
  ns.concat %cat1 %A %U : Tensor[5, 4] float32 // concat() axis=0
  ns.scatter %sc2 %cat1 %U : Tensor[5, 4] float32 // scatter() axis=0 idx=4,0
  ns.slice %sl3 %sc2 : Tensor[3, 4] float32 // slice() axis=0 start=1 stop=4
  ns.transpose %tp4 %sl3 : Tensor[4, 3] float32 // transpose()
  ns.index %ix5 %sc2 : Tensor[3, 4] float32 // index() axis=0 idx=2,2,0
  ns.activation.softmax %f6 %mm0 // softmax()
  ns.reshape %rs7 %f6 : Tensor[0, 6] float32 // reshape() shape=0:6
  ns.concat %cat8 %rs7 %x : Tensor[B, 10] float32 // concat() axis=1
  ns.matmul %mm9 %x %tp4 : Tensor[B, 3] float32 // x @ tp4
  ns.concat %cat10 %cat8 %mm9 : Tensor[B, 13] float32 // concat() axis=1
  ns.index %ix11 %cat10 : Tensor[B, 6] float32 // index() axis=1 idx=12,0,7,3,10,5
  ns.return %ix11
}
