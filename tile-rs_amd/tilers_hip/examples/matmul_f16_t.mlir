module {
  llvm.func @matmul_t_f16(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %m = llvm.mlir.constant(128 : i32) : i32
    %k = llvm.mlir.constant(320 : i32) : i32
    %n = llvm.mlir.constant(264 : i32) : i32
    %a = llvm.call @__tile_load_f16(%arg0, %m, %k) : (!llvm.ptr<1>, i32, i32) -> i32
    %b = llvm.call @__tile_load_f16(%arg1, %n, %k) : (!llvm.ptr<1>, i32, i32) -> i32
    %c = llvm.call @__tile_matmul_transposed_f16(%a, %a, %b, %m, %k, %n) : (i32, i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f16(%arg2, %c, %m, %n) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
  llvm.func @matmul_t_f16_tiles(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %m = llvm.mlir.constant(256 : i32) : i32
    %k = llvm.mlir.constant(512 : i32) : i32
    %n = llvm.mlir.constant(768 : i32) : i32
    %a = llvm.call @__tile_load_f16(%arg0, %m, %k) : (!llvm.ptr<1>, i32, i32) -> i32
    %b = llvm.call @__tile_load_f16(%arg1, %n, %k) : (!llvm.ptr<1>, i32, i32) -> i32
    %c = llvm.call @__tile_matmul_transposed_f16(%a, %a, %b, %m, %k, %n) : (i32, i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f16(%arg2, %c, %m, %n) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
