module {
  llvm.func @swiglu_gate_bf16(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>, %arg3: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %m = llvm.mlir.constant(256 : i32) : i32
    %k = llvm.mlir.constant(512 : i32) : i32
    %n = llvm.mlir.constant(256 : i32) : i32
    %x = llvm.call @__tile_load_f16(%arg0, %m, %k) : (!llvm.ptr<1>, i32, i32) -> i32
    %w = llvm.call @__tile_load_f16(%arg1, %k, %n) : (!llvm.ptr<1>, i32, i32) -> i32
    %g = llvm.call @__tile_matmul_f16(%x, %x, %w, %m, %k, %n) : (i32, i32, i32, i32, i32, i32) -> i32
    %s = llvm.call @__tile_silu_f32(%g, %g, %m, %n) : (i32, i32, i32, i32) -> i32
    %u = llvm.call @__tile_load_f32(%arg2, %m, %n) : (!llvm.ptr<1>, i32, i32) -> i32
    %h = llvm.call @__tile_mul_f32(%s, %s, %u, %m, %n) : (i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg3, %h, %m, %n) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
  llvm.func @swiglu_gate_f16(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>, %arg3: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %m = llvm.mlir.constant(256 : i32) : i32
    %k = llvm.mlir.constant(512 : i32) : i32
    %n = llvm.mlir.constant(512 : i32) : i32
    %x = llvm.call @__tile_load_f16(%arg0, %m, %k) : (!llvm.ptr<1>, i32, i32) -> i32
    %w = llvm.call @__tile_load_f16(%arg1, %k, %n) : (!llvm.ptr<1>, i32, i32) -> i32
    %g = llvm.call @__tile_matmul_f16(%x, %x, %w, %m, %k, %n) : (i32, i32, i32, i32, i32, i32) -> i32
    %s = llvm.call @__tile_silu_f16(%g, %g, %m, %n) : (i32, i32, i32, i32) -> i32
    %u = llvm.call @__tile_load_f16(%arg2, %m, %n) : (!llvm.ptr<1>, i32, i32) -> i32
    %h = llvm.call @__tile_mul_f16(%s, %s, %u, %m, %n) : (i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f16(%arg3, %h, %m, %n) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
