module {
  llvm.func @tile_matmul_transposed(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %m = llvm.mlir.constant(16 : i32) : i32
    %k = llvm.mlir.constant(64 : i32) : i32
    %n = llvm.mlir.constant(16 : i32) : i32
    %a = llvm.call @__tile_load_f32(%arg0, %m, %k) : (!llvm.ptr<1>, i32, i32) -> i32
    %b = llvm.call @__tile_load_f32(%arg1, %n, %k) : (!llvm.ptr<1>, i32, i32) -> i32
    %c = llvm.call @__tile_matmul_transposed_f32(%a, %a, %b, %m, %k, %n) : (i32, i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg2, %c, %m, %n) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
