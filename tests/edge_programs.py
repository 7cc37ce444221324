"""dot_general programs whose shapes are not multiples of the MFMA tiles (partial edge tiles, a K that ends inside a
k-tile) or whose lhs is m-contiguous: the edge instantiations of the MFMA kernels. Used by the CPU plan tests and the
GPU parity tests."""
import numpy as np

from ryft_amd import configs, hostdata as hd, pjrt

_BT = {"bf16": pjrt.BufferType.BF16, "f32": pjrt.BufferType.F32, "i8": pjrt.BufferType.S8,
       "f8E4M3FN": pjrt.BufferType.F8E4M3FN, "f16": pjrt.BufferType.F16}


def _t(shape, dt):
    return "tensor<" + "".join(f"{d}x" for d in shape) + dt + ">"


def _input(seed, shape, dt):
    if dt == "i8":
        return configs.HostInput(hd.int_uniform(seed, shape, -127, 127).astype(np.int8), _BT[dt], shape)
    x = hd.normal(seed, shape, 0.0, 0.5)
    if dt == "bf16":
        return configs.HostInput(hd.f32_to_bf16_bits(x), _BT[dt], shape)
    if dt == "f8E4M3FN":
        return configs.HostInput(hd.f32_to_e4m3fn_bits(x), _BT[dt], shape)
    if dt == "f16":
        return configs.HostInput(x.astype(np.float16).view(np.uint16), _BT[dt], shape)  # raw bits, like bf16
    return configs.HostInput(x.astype(np.float32), _BT[dt], shape)


def dot(name, lhs_shape, rhs_shape, dt, out_dt, lc, rc, lb=(), rb=(), rhs_dt=None, out_convert=None, seed=0):
    """(name, program, inputs, expected kernel family) for one dot_general (+ optional convert of the result)."""
    rhs_dt = rhs_dt or dt
    free_l = [d for i, d in enumerate(lhs_shape) if i not in lc and i not in lb]
    free_r = [d for i, d in enumerate(rhs_shape) if i not in rc and i not in rb]
    out_shape = [lhs_shape[i] for i in lb] + free_l + free_r
    L, R, O = _t(lhs_shape, dt), _t(rhs_shape, rhs_dt), _t(out_shape, out_dt)
    bd = f"batching_dims = [{', '.join(map(str, lb))}] x [{', '.join(map(str, rb))}], " if lb else ""
    body = (f"    %0 = stablehlo.dot_general %arg0, %arg1, {bd}contracting_dims = [{', '.join(map(str, lc))}] x "
            f"[{', '.join(map(str, rc))}] : ({L}, {R}) -> {O}\n")
    ret, rty = "%0", O
    if out_convert:
        rty = _t(out_shape, out_convert)
        body += f"    %1 = stablehlo.convert %0 : ({O}) -> {rty}\n"
        ret = "%1"
    prog = (f"module {{\n  func.func @main(%arg0: {L}, %arg1: {R}) -> {rty} {{\n{body}    return {ret} : {rty}\n"
            f"  }}\n}}\n")
    ins = [_input(seed * 2 + 1, tuple(lhs_shape), dt), _input(seed * 2 + 2, tuple(rhs_shape), rhs_dt)]
    return name, prog, ins


CASES = [
    # (case, expected kernel, tolerance)
    (dot("bf16_ragged_mnk", (1000, 1000), (1000, 1008), "bf16", "f32", [1], [0], out_convert="bf16", seed=1),
     "gemm_bf16_mfma_edge_128x128", 1e-2),
    (dot("bf16_m_contiguous_lhs", (256, 296), (256, 128), "bf16", "f32", [0], [0], seed=2),
     "gemm_bf16_mfma_edge_128x128", 1e-2),
    (dot("bf16_batched_ragged", (3, 100, 72), (3, 72, 48), "bf16", "f32", [2], [1], [0], [0], seed=3),
     "gemm_bf16_mfma_edge_128x128", 1e-2),
    (dot("bf16_k_contiguous_rhs", (130, 200), (272, 200), "bf16", "f32", [1], [1], seed=4),
     "gemm_bf16_mfma_edge_128x128", 1e-2),
    (dot("i8_ragged_k_tail", (300, 528), (528, 272), "i8", "i32", [1], [0], seed=5),
     "gemm_i8_mfma_edge_128x128", 0.0),
    (dot("i8_m_contiguous_lhs", (256, 208), (256, 96), "i8", "i32", [0], [0], seed=6),
     "gemm_i8_mfma_edge_128x128", 0.0),
    (dot("f32_ragged", (250, 100), (100, 96), "f32", "f32", [1], [0], seed=7),
     "gemm_f32_mfma_edge_64x64", 1e-4),
    (dot("fp8_ragged", (200, 272), (272, 160), "f8E4M3FN", "f32", [1], [0], seed=8),
     "gemm_fp8_mfma_edge_128x128", 1e-2),
    (dot("bf16_f8_ragged", (100, 264), (264, 400), "bf16", "f32", [1], [0], rhs_dt="f8E4M3FN", seed=9),
     "gemm_bf16f8_mfma_edge_128x128", 1e-2),
    (dot("bf16_f8_k_contiguous_rhs", (100, 264), (400, 264), "bf16", "f32", [1], [1], rhs_dt="f8E4M3FN", seed=10),
     "gemm_bf16f8_mfma_edge_128x128", 1e-2),
    (dot("f16_ragged", (136, 200), (200, 80), "f16", "f32", [1], [0], seed=11),
     "gemm_f16_mfma_edge_128x128", 1e-2),
    # N not a multiple of 16: partial output chunks stored an element at a time; rhs rows that are not 16-byte
    # aligned (n-contiguous N·size % 16 != 0) copied into padded rows first
    (dot("bf16_n1000", (1000, 1000), (1000, 1000), "bf16", "f32", [1], [0], out_convert="bf16", seed=12),
     "gemm_bf16_mfma_edge_128x128", 1e-2),
    (dot("bf16_n100_unaligned_rhs", (512, 4096), (4096, 100), "bf16", "f32", [1], [0], seed=13),
     "gemm_bf16_mfma_edge_128x128", 1e-2),
    (dot("f32_n250_unaligned_rhs", (256, 512), (512, 250), "f32", "f32", [1], [0], seed=14),
     "gemm_f32_mfma_edge_64x64", 1e-4),
    (dot("i8_n4008_unaligned_rhs", (4096, 4096), (4096, 4008), "i8", "i32", [1], [0], seed=15),
     "gemm_i8_mfma_edge_128x128", 0.0),
    (dot("bf16_odd_n37_k99", (64, 99), (99, 37), "bf16", "f32", [1], [0], out_convert="bf16", seed=16),
     "gemm_bf16_mfma_edge_128x128", 1e-2),
    (dot("fp8_n40", (96, 256), (256, 40), "f8E4M3FN", "f32", [1], [0], seed=17),
     "gemm_fp8_mfma_edge_128x128", 1e-2),
    (dot("bf16_f8_n72", (100, 264), (264, 72), "bf16", "f32", [1], [0], rhs_dt="f8E4M3FN", seed=18),
     "gemm_bf16f8_mfma_edge_128x128", 1e-2),
    (dot("f16_k_contiguous_n24", (80, 64), (24, 64), "f16", "f32", [1], [1], seed=19),
     "gemm_f16_mfma_edge_128x128", 1e-2),
]
