// NeuralScript MLIR
ns.func @DMX {
  ns.tensor.alloc %W : Tensor[3, 5] float32 // allocate Tensor[3, 5] float32
  ns.tensor.alloc %V : Tensor[5, 7] float32 // allocate Tensor[5, 7] float32
  ns.concat %cat0 %x %x : Tensor[B, 10] float32 // concat() axis=1
  ns.transpose %tp1 %W : Tensor[5, 3] float32 // transpose()
  ns.slice %sl2 %cat0 : Tensor[2, 10] float32 // slice() axis=0 start=1 stop=3
  ns.matmul %mm3 %x %V : Tensor[B, 7] float32 // x @ V
  ns.slice %sl4 %cat0 : Tensor[B, 7] float32 // slice() axis=1 start=2 stop=9
  ns.index %ix5 %sl4 : Tensor[B, 3] float32 // index() axis=1 idx=6,0,3
  ns.scatter %sc6 %sl4 %ix5 : Tensor[B, 7] float32 // scatter() axis=1 idx=1,5,1
  ns.return %sc6
}
