module {
  llvm.func @tile_sample_top_p(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %rows  = llvm.mlir.constant(4 : i32) : i32
    %cols  = llvm.mlir.constant(256 : i32) : i32
    %temp  = llvm.mlir.constant(1 : i32) : i32
    %topp  = llvm.mlir.constant(0 : i32) : i32
    %seed  = llvm.mlir.constant(42 : i32) : i32
    %src = llvm.call @__tile_load_f32(%arg0, %rows, %cols) : (!llvm.ptr<1>, i32, i32) -> i32
    %res = llvm.call @__tile_sample_top_p_f32(%src, %src, %temp, %topp, %seed, %rows, %cols) : (i32, i32, i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg1, %res, %rows, %cols) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
