module {
  llvm.func @tile_fill(%arg0: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %r = llvm.mlir.constant(1 : i32) : i32
    %c = llvm.mlir.constant(1024 : i32) : i32
    %v = llvm.mlir.constant(3.500000e+00 : f32) : f32
    %y = llvm.call @__tile_fill_f32(%r, %v, %r, %c) : (i32, f32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg0, %y, %r, %c) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
