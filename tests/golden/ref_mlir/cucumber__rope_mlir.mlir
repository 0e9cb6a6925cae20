module {
  llvm.func @rope_test(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %rows = llvm.mlir.constant(4 : i32) : i32
    %cols = llvm.mlir.constant(64 : i32) : i32
    %pos  = llvm.mlir.constant(7 : i32) : i32
    %a = llvm.call @__tile_load_f32(%arg0, %rows, %cols) : (!llvm.ptr<1>, i32, i32) -> i32
    %res = llvm.call @__tile_rope_f32(%a, %a, %pos, %rows, %cols) : (i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg1, %res, %rows, %cols) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
