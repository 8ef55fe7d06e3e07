// NeuralScript MLIR
ns.func @DMV {
  ns.tensor.alloc %W : Tensor[5, 6] float32 // allocate Tensor[5, 6] float32
  ns.tensor.alloc %V : Tensor[6, 4] float32 // allocate Tensor[6, 4] float32
  ns.matmul %mm0 %x %V : Tensor[B, 4] float32 // x @ V
  ns.concat %cat1 %mm0 %x : Tensor[B, 10] float32 // concat() axis=1
  ns.slice %sl2 %cat1 : Tensor[B, 6] float32 // slice() axis=1 start=2 stop=8
  ns.index %ix3 %cat1 : Tensor[B, 3] float32 // index() axis=1 idx=9,0,4
  ns.index %ix4 %W : Tensor[2, 6] float32 // index() axis=0 idx=4,1
  ns.transpose %tp5 %W : Tensor[6, 5] float32 // transpose()
  ns.scatter %sc6 %cat1 %ix3 : Tensor[B, 10] float32 // scatter() axis=1 idx=1,3,5
  ns.slice %sl7 %sc6 : Tensor[B, 9] float32 // slice() axis=1 start=1 stop=10
  ns.return %sl7
}
