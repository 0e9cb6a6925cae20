module {
  llvm.func @tile_clamp(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %1 = llvm.mlir.constant(1 : i32) : i32
    %2 = llvm.mlir.constant(256 : i32) : i32
    %min = llvm.mlir.constant(0 : i32) : i32
    %max = llvm.mlir.constant(6 : i32) : i32
    %3 = llvm.call @__tile_load_f32(%arg0, %1, %2) : (!llvm.ptr<1>, i32, i32) -> i32
    %4 = llvm.call @__tile_clamp_f32(%3, %3, %min, %max, %1, %2) : (i32, i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg1, %4, %1, %2) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
