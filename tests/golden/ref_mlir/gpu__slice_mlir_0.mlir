module {
  llvm.func @tile_slice(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %ro = llvm.mlir.constant(2 : i32) : i32
    %co = llvm.mlir.constant(4 : i32) : i32
    %sr = llvm.mlir.constant(16 : i32) : i32
    %sc = llvm.mlir.constant(32 : i32) : i32
    %dr = llvm.mlir.constant(8 : i32) : i32
    %dc = llvm.mlir.constant(16 : i32) : i32
    %5 = llvm.call @__tile_slice_f32(%arg0, %arg0, %ro, %co, %sr, %sc, %dr, %dc) : (!llvm.ptr<1>, !llvm.ptr<1>, i32, i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg1, %5, %dr, %dc) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
