module {
  "llvm.func"() <{function_type = !llvm.func<void (ptr<1>, ptr<1>)>, sym_name = "softmax_loop_bf16_generic"}> ({
  ^bb0(%arg0: !llvm.ptr<1>, %arg1: !llvm.ptr<1>):
    %0 = "llvm.mlir.constant"() <{value = 1 : i32}> : () -> i32
    "llvm.call"(%0) <{callee = @__tile_pipelined_for_begin, fastmathFlags = #llvm.fastmath<none>}> : (i32) -> ()
    %1 = "llvm.mlir.constant"() <{value = 0 : i32}> : () -> i32
    %2 = "llvm.mlir.constant"() <{value = 4 : i32}> : () -> i32
    %3 = "llvm.mlir.constant"() <{value = 512 : i32}> : () -> i32
    %4 = "llvm.mlir.constant"() <{value = 2048 : i32}> : () -> i32
    %5 = "llvm.mlir.constant"() <{value = 48 : i32}> : () -> i32
    "llvm.br"(%1)[^bb1] : (i32) -> ()
  ^bb1(%6: i32):
    %7 = "llvm.icmp"(%6, %5) <{predicate = 9 : i64}> : (i32, i32) -> i1
    "llvm.cond_br"(%7)[^bb3, ^bb2] <{operandSegmentSizes = array<i32: 1, 0, 0>}> : (i1) -> ()
  ^bb2:
    %8 = "llvm.mul"(%6, %4) <{overflowFlags = #llvm.overflow<none>}> : (i32, i32) -> i32
    %9 = "llvm.zext"(%8) : (i32) -> i64
    %10 = "llvm.getelementptr"(%arg0, %9) <{elem_type = i16, rawConstantIndices = array<i32: -2147483648>}> : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>
    %11 = "llvm.getelementptr"(%arg1, %9) <{elem_type = i16, rawConstantIndices = array<i32: -2147483648>}> : (!llvm.ptr<1>, i64) -> !llvm.ptr<1>
    %12 = "llvm.call"(%10, %2, %3) <{callee = @__tile_load_f16, fastmathFlags = #llvm.fastmath<none>}> : (!llvm.ptr<1>, i32, i32) -> i32
    %13 = "llvm.call"(%12, %12, %2, %3) <{callee = @__tile_softmax_f16, fastmathFlags = #llvm.fastmath<none>}> : (i32, i32, i32, i32) -> i32
    "llvm.call"(%11, %13, %2, %3) <{callee = @__tile_store_f16, fastmathFlags = #llvm.fastmath<none>}> : (!llvm.ptr<1>, i32, i32, i32) -> ()
    %14 = "llvm.mlir.constant"() <{value = 1 : i32}> : () -> i32
    %15 = "llvm.add"(%6, %14) <{overflowFlags = #llvm.overflow<none>}> : (i32, i32) -> i32
    "llvm.br"(%15)[^bb1] : (i32) -> ()
  ^bb3:
    "llvm.call"() <{callee = @__tile_pipelined_for_end, fastmathFlags = #llvm.fastmath<none>}> : () -> ()
    "llvm.return"() : () -> ()
  }) {hacc.entry} : () -> ()
}
