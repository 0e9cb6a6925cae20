module {
  llvm.func @tile_token_accept(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>, %arg3: !llvm.ptr<1>, %arg4: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %rows   = llvm.mlir.constant(8 : i32) : i32
    %cols   = llvm.mlir.constant(1 : i32) : i32
    %thresh = llvm.mlir.constant(0 : i32) : i32
    %draft  = llvm.call @__tile_load_f32(%arg0, %rows, %cols) : (!llvm.ptr<1>, i32, i32) -> i32
    %target = llvm.call @__tile_load_f32(%arg1, %rows, %cols) : (!llvm.ptr<1>, i32, i32) -> i32
    %probs  = llvm.call @__tile_load_f32(%arg2, %rows, %cols) : (!llvm.ptr<1>, i32, i32) -> i32
    %res = llvm.call @__tile_token_accept_f32(%probs, %draft, %target, %probs, %thresh, %rows) : (i32, i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg4, %res, %rows, %cols) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
