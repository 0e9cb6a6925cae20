module {
  llvm.func @gemm_loop_bf16(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>, %arg3: i32) attributes {hacc.entry} {
    ^bb0:
    %depth = llvm.mlir.constant(5 : i32) : i32
    llvm.call @__tile_pipelined_for_begin(%depth) : (i32) -> ()
    %zero = llvm.mlir.constant(0 : i32) : i32
    %one = llvm.mlir.constant(1 : i32) : i32
    %m = llvm.mlir.constant(256 : i32) : i32
    %k = llvm.mlir.constant(320 : i32) : i32
    %n = llvm.mlir.constant(384 : i32) : i32
    %mk = llvm.mlir.constant(81920 : i64) : i64
    %kn = llvm.mlir.constant(122880 : i64) : i64
    %mn = llvm.mlir.constant(98304 : i64) : i64
    llvm.br ^bb1(%zero : i32)
  ^bb1(%i: i32):
    %done = llvm.icmp "uge" %i, %arg3 : i32
    llvm.cond_br %done, ^bb3, ^bb2
  ^bb2:
    %iw = llvm.zext %i : i32 to i64
    %oa = llvm.mul %iw, %mk : i64
    %ob = llvm.mul %iw, %kn : i64
    %oc = llvm.mul %iw, %mn : i64
    %pa = llvm.getelementptr %arg0[%oa] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, i16
    %pb = llvm.getelementptr %arg1[%ob] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, i16
    %pc = llvm.getelementptr %arg2[%oc] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, f32
    %a = llvm.call @__tile_load_f16(%pa, %m, %k) : (!llvm.ptr<1>, i32, i32) -> i32
    %b = llvm.call @__tile_load_f16(%pb, %k, %n) : (!llvm.ptr<1>, i32, i32) -> i32
    %c = llvm.call @__tile_matmul_f16(%a, %a, %b, %m, %k, %n) : (i32, i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%pc, %c, %m, %n) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    %next = llvm.add %i, %one : i32
    llvm.br ^bb1(%next : i32)
  ^bb3:
    llvm.call @__tile_pipelined_for_end() : () -> ()
    llvm.return
  }
}
