module {
  llvm.func @rope_f32(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %rows = llvm.mlir.constant(4 : i32) : i32
    %cols = llvm.mlir.constant(64 : i32) : i32
    %pos = llvm.mlir.constant(7 : i32) : i32
    %x = llvm.call @__tile_load_f32(%arg0, %rows, %cols) : (!llvm.ptr<1>, i32, i32) -> i32
    %y = llvm.call @__tile_rope_f32(%x, %x, %pos, %rows, %cols) : (i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg1, %y, %rows, %cols) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
  llvm.func @rope_bf16(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %rows = llvm.mlir.constant(2 : i32) : i32
    %cols = llvm.mlir.constant(128 : i32) : i32
    %pos = llvm.mlir.constant(1000 : i32) : i32
    %x = llvm.call @__tile_load_f16(%arg0, %rows, %cols) : (!llvm.ptr<1>, i32, i32) -> i32
    %y = llvm.call @__tile_rope_f16(%x, %x, %pos, %rows, %cols) : (i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f16(%arg1, %y, %rows, %cols) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
