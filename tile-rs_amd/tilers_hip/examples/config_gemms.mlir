module {
  llvm.func @gemm_4096_bf16_acc_f32(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %m = llvm.mlir.constant(4096 : i32) : i32
    %k = llvm.mlir.constant(4096 : i32) : i32
    %n = llvm.mlir.constant(4096 : i32) : i32
    %a = llvm.call @__tile_load_f16(%arg0, %m, %k) : (!llvm.ptr<1>, i32, i32) -> i32
    %b = llvm.call @__tile_load_f16(%arg1, %k, %n) : (!llvm.ptr<1>, i32, i32) -> i32
    %c = llvm.call @__tile_matmul_f16(%a, %a, %b, %m, %k, %n) : (i32, i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg2, %c, %m, %n) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
  llvm.func @mlp_up_f16(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %m = llvm.mlir.constant(8192 : i32) : i32
    %k = llvm.mlir.constant(4096 : i32) : i32
    %n = llvm.mlir.constant(14336 : i32) : i32
    %a = llvm.call @__tile_load_f16(%arg0, %m, %k) : (!llvm.ptr<1>, i32, i32) -> i32
    %b = llvm.call @__tile_load_f16(%arg1, %k, %n) : (!llvm.ptr<1>, i32, i32) -> i32
    %c = llvm.call @__tile_matmul_f16(%a, %a, %b, %m, %k, %n) : (i32, i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f16(%arg2, %c, %m, %n) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
  llvm.func @mlp_gate_f16(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>, %arg3: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %m = llvm.mlir.constant(8192 : i32) : i32
    %k = llvm.mlir.constant(4096 : i32) : i32
    %n = llvm.mlir.constant(14336 : i32) : i32
    %a = llvm.call @__tile_load_f16(%arg0, %m, %k) : (!llvm.ptr<1>, i32, i32) -> i32
    %b = llvm.call @__tile_load_f16(%arg1, %k, %n) : (!llvm.ptr<1>, i32, i32) -> i32
    %g = llvm.call @__tile_matmul_f16(%a, %a, %b, %m, %k, %n) : (i32, i32, i32, i32, i32, i32) -> i32
    %s = llvm.call @__tile_silu_f16(%g, %g, %m, %n) : (i32, i32, i32, i32) -> i32
    %u = llvm.call @__tile_load_f16(%arg2, %m, %n) : (!llvm.ptr<1>, i32, i32) -> i32
    %h = llvm.call @__tile_mul_f16(%s, %s, %u, %m, %n) : (i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f16(%arg3, %h, %m, %n) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
