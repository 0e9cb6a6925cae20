module {
  llvm.func @tile_concat(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %rows = llvm.mlir.constant(4 : i32) : i32
    %ca = llvm.mlir.constant(8 : i32) : i32
    %cb = llvm.mlir.constant(16 : i32) : i32
    %5 = llvm.call @__tile_concat_f32(%arg0, %arg1, %arg2, %rows, %ca, %cb) : (!llvm.ptr<1>, !llvm.ptr<1>, !llvm.ptr<1>, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg0, %5, %rows, %ca) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
