module {
  llvm.func @softmax_loop_f32(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: i32) attributes {hacc.entry} {
    ^bb0:
    %depth = llvm.mlir.constant(2 : i32) : i32
    llvm.call @__tile_pipelined_for_begin(%depth) : (i32) -> ()
    %zero = llvm.mlir.constant(0 : i32) : i32
    %one = llvm.mlir.constant(1 : i32) : i32
    %cols = llvm.mlir.constant(1024 : i32) : i32
    %cols64 = llvm.mlir.constant(1024 : i64) : i64
    llvm.br ^bb1(%zero : i32)
  ^bb1(%i: i32):
    %done = llvm.icmp "uge" %i, %arg2 : i32
    llvm.cond_br %done, ^bb3, ^bb2
  ^bb2:
    %iw = llvm.zext %i : i32 to i64
    %off = llvm.mul %iw, %cols64 : i64
    %src = llvm.getelementptr %arg0[%off] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, f32
    %dst = llvm.getelementptr %arg1[%off] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, f32
    %t = llvm.call @__tile_load_f32(%src, %one, %cols) : (!llvm.ptr<1>, i32, i32) -> i32
    %y = llvm.call @__tile_softmax_f32(%t, %t, %one, %cols) : (i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%dst, %y, %one, %cols) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    %next = llvm.add %i, %one : i32
    llvm.br ^bb1(%next : i32)
  ^bb3:
    llvm.call @__tile_pipelined_for_end() : () -> ()
    llvm.return
  }
  llvm.func @add_loop_f32(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: !llvm.ptr<1>, %arg3: i64) attributes {hacc.entry} {
    ^bb0:
    %zero = llvm.mlir.constant(0 : i64) : i64
    %one = llvm.mlir.constant(1 : i64) : i64
    %r = llvm.mlir.constant(2 : i32) : i32
    %c = llvm.mlir.constant(256 : i32) : i32
    %step = llvm.mlir.constant(9 : i64) : i64
    llvm.br ^bb1(%zero : i64)
  ^bb1(%i: i64):
    %more = llvm.icmp "ult" %i, %arg3 : i64
    llvm.cond_br %more, ^bb2, ^bb3
  ^bb2:
    %off = llvm.shl %i, %step : i64
    %pa = llvm.getelementptr %arg0[%off] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, f32
    %pb = llvm.getelementptr %arg1[%off] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, f32
    %pc = llvm.getelementptr %arg2[%off] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, f32
    %a = llvm.call @__tile_load_f32(%pa, %r, %c) : (!llvm.ptr<1>, i32, i32) -> i32
    %b = llvm.call @__tile_load_f32(%pb, %r, %c) : (!llvm.ptr<1>, i32, i32) -> i32
    %s = llvm.call @__tile_add_f32(%a, %a, %b, %r, %c) : (i32, i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%pc, %s, %r, %c) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    %next = llvm.add %one, %i : i64
    llvm.br ^bb1(%next : i64)
  ^bb3:
    llvm.return
  }
  llvm.func @softmax_loop_signed_f32(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>, %arg2: i32) attributes {hacc.entry} {
    ^bb0:
    %zero = llvm.mlir.constant(0 : i32) : i32
    %one = llvm.mlir.constant(1 : i32) : i32
    %cols = llvm.mlir.constant(1024 : i32) : i32
    %cols64 = llvm.mlir.constant(1024 : i64) : i64
    llvm.br ^bb1(%zero : i32)
  ^bb1(%i: i32):
    %more = llvm.icmp "slt" %i, %arg2 : i32
    llvm.cond_br %more, ^bb2, ^bb3
  ^bb2:
    %iw = llvm.zext %i : i32 to i64
    %off = llvm.mul %iw, %cols64 : i64
    %src = llvm.getelementptr %arg0[%off] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, f32
    %dst = llvm.getelementptr %arg1[%off] : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>, f32
    %t = llvm.call @__tile_load_f32(%src, %one, %cols) : (!llvm.ptr<1>, i32, i32) -> i32
    %y = llvm.call @__tile_softmax_f32(%t, %t, %one, %cols) : (i32, i32, i32, i32) -> i32
    llvm.call @__tile_store_f32(%dst, %y, %one, %cols) : (!llvm.ptr<1>, i32, i32, i32) -> ()
    %next = llvm.add %i, %one : i32
    llvm.br ^bb1(%next : i32)
  ^bb3:
    llvm.return
  }
}
