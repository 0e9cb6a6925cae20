module {
  llvm.func @simple_copy(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %1 = llvm.mlir.constant(1 : i32) : i32
    %2 = llvm.mlir.constant(1024 : i32) : i32
    %3 = llvm.call @__tile_load_f32(%arg0, %1, %2) : (!llvm.ptr<1>, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg1, %3, %1, %2) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
