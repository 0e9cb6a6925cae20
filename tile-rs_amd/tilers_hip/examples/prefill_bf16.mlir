module {
  llvm.func @prefill_bf16(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>, %arg3: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %nh = llvm.mlir.constant(32 : i32) : i32
    %dh = llvm.mlir.constant(128 : i32) : i32
    %q = llvm.call @__tile_load_f16(%arg0, %nh, %dh) : (!llvm.ptr<1>, i32, i32) -> i32
    %k = llvm.call @__tile_load_f16(%arg1, %nh, %dh) : (!llvm.ptr<1>, i32, i32) -> i32
    %v = llvm.call @__tile_load_f16(%arg2, %nh, %dh) : (!llvm.ptr<1>, i32, i32) -> i32
    %o = llvm.call @__tile_attention_prefill_f32(%q, %q, %k, %v, %nh, %dh) : (i32, i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f16(%arg3, %o, %nh, %dh) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
