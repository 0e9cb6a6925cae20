module {
  llvm.func @attention_gqa_f32(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>, %arg3: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %nh = llvm.mlir.constant(8 : i32) : i32
    %nkv = llvm.mlir.constant(2 : i32) : i32
    %seq = llvm.mlir.constant(32 : i32) : i32
    %hd = llvm.mlir.constant(64 : i32) : i32
    %q = llvm.call @__tile_load_f32(%arg0, %nh, %seq) : (!llvm.ptr<1>, i32, i32) -> i32
    %k = llvm.call @__tile_load_f32(%arg1, %nkv, %seq) : (!llvm.ptr<1>, i32, i32) -> i32
    %v = llvm.call @__tile_load_f32(%arg2, %nkv, %seq) : (!llvm.ptr<1>, i32, i32) -> i32
    %out = llvm.call @__tile_attention_gqa_f32(%q, %q, %k, %v, %nh, %nkv, %seq, %hd) : (i32, i32, i32, i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg3, %out, %nh, %seq) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
  llvm.func @attention_gqa_wide_f32(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>, %arg3: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %nh = llvm.mlir.constant(4 : i32) : i32
    %nkv = llvm.mlir.constant(1 : i32) : i32
    %seq = llvm.mlir.constant(1500 : i32) : i32
    %hd = llvm.mlir.constant(96 : i32) : i32
    %q = llvm.call @__tile_load_f32(%arg0, %nh, %seq) : (!llvm.ptr<1>, i32, i32) -> i32
    %k = llvm.call @__tile_load_f32(%arg1, %nkv, %seq) : (!llvm.ptr<1>, i32, i32) -> i32
    %v = llvm.call @__tile_load_f32(%arg2, %nkv, %seq) : (!llvm.ptr<1>, i32, i32) -> i32
    %out = llvm.call @__tile_attention_gqa_f32(%q, %q, %k, %v, %nh, %nkv, %seq, %hd) : (i32, i32, i32, i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg3, %out, %nh, %seq) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
  llvm.func @attention_gqa_bf16(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>, %arg3: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %nh = llvm.mlir.constant(8 : i32) : i32
    %nkv = llvm.mlir.constant(2 : i32) : i32
    %seq = llvm.mlir.constant(300 : i32) : i32
    %hd = llvm.mlir.constant(128 : i32) : i32
    %q = llvm.call @__tile_load_f16(%arg0, %nh, %seq) : (!llvm.ptr<1>, i32, i32) -> i32
    %k = llvm.call @__tile_load_f16(%arg1, %nkv, %seq) : (!llvm.ptr<1>, i32, i32) -> i32
    %v = llvm.call @__tile_load_f16(%arg2, %nkv, %seq) : (!llvm.ptr<1>, i32, i32) -> i32
    %out = llvm.call @__tile_attention_gqa_f16(%q, %q, %k, %v, %nh, %nkv, %seq, %hd) : (i32, i32, i32, i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f16(%arg3, %out, %nh, %seq) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
