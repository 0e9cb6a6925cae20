module {
  llvm.func @swiglu(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %r = llvm.mlir.constant(2 : i32) : i32
    %c = llvm.mlir.constant(64 : i32) : i32
    %gate = llvm.call @__tile_load_f32(%arg0, %r, %c) : (!llvm.ptr<1>, i32, i32) -> i32
    %up = llvm.call @__tile_load_f32(%arg1, %r, %c) : (!llvm.ptr<1>, i32, i32) -> i32
    %s = llvm.call @__tile_silu_f32(%gate, %gate, %r, %c) : (i32, i32, i32, i32) -> i32
    %res = llvm.call @__tile_mul_f32(%s, %s, %up, %r, %c) : (i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg2, %res, %r, %c) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
  llvm.func @scaled_causal(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>) attributes {hacc.entry} {
    ^bb0:
    %s = llvm.mlir.constant(16 : i32) : i32
    %f = llvm.mlir.constant(1.250000e-01 : f32) : f32
    %lo = llvm.mlir.constant(-4.000000e+00 : f32) : f32
    %hi = llvm.mlir.constant(4.000000e+00 : f32) : f32
    %x = llvm.call @__tile_load_f32(%arg0, %s, %s) : (!llvm.ptr<1>, i32, i32) -> i32
    %y = llvm.call @__tile_scale_f32(%x, %x, %f, %s, %s) : (i32, i32, f32, i32, i32) -> i32
    %z = llvm.call @__tile_clamp_f32(%y, %y, %lo, %hi, %s, %s) : (i32, i32, f32, f32, i32, i32) -> i32
    %m = llvm.call @__tile_causal_mask_f32(%z, %z, %s, %s) : (i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%arg1, %m, %s, %s) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    llvm.return
  }
}
