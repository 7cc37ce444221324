"""StableHLO programs with input/output aliasing (func argument attributes `tf.aliasing_output` and
`jax.buffer_donor`), as XLA's aliasing guide describes them and ryft-pjrt's ExecutionInput::donatable
(crates/ryft-pjrt/src/programs.rs:1003-1016) exercises them: a parameter donated to a result of the same type."""

N = 1 << 16

# an optimizer-style update: the donated parameter is read only at the element each thread writes → in place
SGD = f"""module {{
  func.func @main(%arg0: tensor<{N}xf32> {{tf.aliasing_output = 0 : i32}}, %arg1: tensor<{N}xf32>) -> tensor<{N}xf32> {{
    %0 = stablehlo.constant dense<0.125> : tensor<{N}xf32>
    %1 = stablehlo.multiply %arg1, %0 : tensor<{N}xf32>
    %2 = stablehlo.subtract %arg0, %1 : tensor<{N}xf32>
    return %2 : tensor<{N}xf32>
  }}
}}
"""

# a GEMM result aliased to its left operand: the operand is read by every output tile → a buffer of its own
GEMM = """module {
  func.func @main(%arg0: tensor<256x256xbf16> {tf.aliasing_output = 0 : i32}, %arg1: tensor<256x256xbf16>) -> tensor<256x256xbf16> {
    %0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1] x [0] : (tensor<256x256xbf16>, tensor<256x256xbf16>) -> tensor<256x256xf32>
    %1 = stablehlo.convert %0 : (tensor<256x256xf32>) -> tensor<256x256xbf16>
    return %1 : tensor<256x256xbf16>
  }
}
"""

# the donated parameter is also read transposed by the step that writes the result → a buffer of its own
TRANSPOSED = """module {
  func.func @main(%arg0: tensor<64x64xf32> {tf.aliasing_output = 0 : i32}) -> tensor<64x64xf32> {
    %0 = stablehlo.transpose %arg0, dims = [1, 0] : (tensor<64x64xf32>) -> tensor<64x64xf32>
    %1 = stablehlo.add %arg0, %0 : tensor<64x64xf32>
    return %1 : tensor<64x64xf32>
  }
}
"""

# a parameter returned unchanged and donated to that result (in place: nothing to copy), next to a computed result
PASSTHROUGH = """module {
  func.func @main(%arg0: tensor<1024xi32> {tf.aliasing_output = 1 : i32}, %arg1: tensor<1024xi32>) -> (tensor<1024xi32>, tensor<1024xi32>) {
    %0 = stablehlo.add %arg0, %arg1 : tensor<1024xi32>
    return %0, %arg0 : tensor<1024xi32>, tensor<1024xi32>
  }
}
"""

# buffer donors: the compiler pairs each with the first unclaimed result of its type (here result 1, the f32 one)
DONOR = """module {
  func.func @main(%arg0: tensor<512xf32> {jax.buffer_donor = true}, %arg1: tensor<512xi32>) -> (tensor<512xi32>, tensor<512xf32>) {
    %0 = stablehlo.add %arg1, %arg1 : tensor<512xi32>
    %1 = stablehlo.exponential %arg0 : tensor<512xf32>
    return %0, %1 : tensor<512xi32>, tensor<512xf32>
  }
}
"""

# malformed aliasing: (program, message fragment)
BAD = {
    "result_out_of_range": ("""module {
  func.func @main(%arg0: tensor<4xf32> {tf.aliasing_output = 1 : i32}) -> tensor<4xf32> {
    %0 = stablehlo.negate %arg0 : tensor<4xf32>
    return %0 : tensor<4xf32>
  }
}
""", "the function has 1 result"),
    "type_mismatch": ("""module {
  func.func @main(%arg0: tensor<4xf32> {tf.aliasing_output = 0 : i32}) -> tensor<4xbf16> {
    %0 = stablehlo.convert %arg0 : (tensor<4xf32>) -> tensor<4xbf16>
    return %0 : tensor<4xbf16>
  }
}
""", "the types differ"),
    "two_parameters_one_result": ("""module {
  func.func @main(%arg0: tensor<4xf32> {tf.aliasing_output = 0 : i32}, %arg1: tensor<4xf32> {tf.aliasing_output = 0 : i32}) -> tensor<4xf32> {
    %0 = stablehlo.add %arg0, %arg1 : tensor<4xf32>
    return %0 : tensor<4xf32>
  }
}
""", "aliased to both parameter 0 and parameter 1"),
}
