module {
  llvm.func @tile_draft_verify(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %rows = llvm.mlir.constant(8 : i32) : i32
    %cols = llvm.mlir.constant(128 : i32) : i32
    %draft = llvm.call @__tile_load_f32(%arg0, %rows, %cols) : (!llvm.ptr<1>, i32, i32) -> i32
    %logits = llvm.call @__tile_load_f32(%arg1, %rows, %cols) : (!llvm.ptr<1>, i32, i32) -> i32
    %res = llvm.call @__tile_draft_verify_f32(%logits, %draft, %logits, %rows, %cols) : (i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg2, %res, %rows, %cols) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
