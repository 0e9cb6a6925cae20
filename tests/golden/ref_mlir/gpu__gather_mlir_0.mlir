module {
  llvm.func @tile_gather(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %n = llvm.mlir.constant(8 : i32) : i32
    %m = llvm.mlir.constant(16 : i32) : i32
    %d = llvm.mlir.constant(32 : i32) : i32
    %5 = llvm.call @__tile_gather_f32(%arg0, %arg1, %arg2, %n, %m, %d) : (!llvm.ptr<1>, !llvm.ptr<1>, !llvm.ptr<1>, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg0, %5, %n, %d) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
