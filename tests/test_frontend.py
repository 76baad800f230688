"""Front end of libtforge_hip on the CPU (tf_compile makes no GPU call).

Restates, as executable checks, the reference's lit tests for the path:
  * test/Dialect/TForge/invalid.mlir -- the 18 verifier diagnostics;
  * test/Pipelines/gpu-pipeline.mlir:21 -- grid/block of the naive kernel;
  * test/Pipelines/gpu-staged.mlir:39 -- the located NOTPADDED error;
  * test/Transforms/gpu-tile-script.mlir:17 -- block dims from the tiles;
  * results/gpu/stage8_ir/.../launch.json, stage7_ir/.../launch.json -- geometry;
  * lib/Pipelines/Pipelines.cpp:214-263 -- option defaults and errors.
"""

import json
import pathlib

import pytest

from tensorforge_amd import _lib
from tensorforge_amd import tforge_cpu as tc
from tensorforge_amd import tforge_gpu as tg

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def compile_err(program, options=""):
    with pytest.raises(RuntimeError) as e:
        _lib.Kernel(program, options, "t.mlir")
    return str(e.value)


# (function body line, expected diagnostic) -- test/Dialect/TForge/invalid.mlir
INVALID = [
    ("%a: f32", '%0 = "tforge.relu"(%a) : (f32) -> tensor<4xf32>',
     "'tforge.relu' op operand #0 must be tensor of any non-token type values, but got 'f32'"),
    ("%a: tensor<*xf32>", "%0 = tforge.add %a, %a : tensor<*xf32>, tensor<*xf32> -> tensor<4xf32>",
     "'tforge.add' op lhs must be a ranked tensor, but got 'tensor<*xf32>'"),
    ("%a: tensor<?x4xf32>", "%0 = tforge.relu %a : tensor<?x4xf32> -> tensor<?x4xf32>",
     "'tforge.relu' op input must have a static shape, but got 'tensor<?x4xf32>'"),
    ("%a: tensor<4xf16>", "%0 = tforge.relu %a : tensor<4xf16> -> tensor<4xf16>",
     "'tforge.relu' op input must have f32 elements, but has element type 'f16'"),
    ("%a: tensor<4xi32>, %b: tensor<4xf32>", "%0 = tforge.add %a, %b : tensor<4xi32>, tensor<4xf32> -> tensor<4xf32>",
     "'tforge.add' op lhs must have f32 elements, but has element type 'i32'"),
    ("%a: tensor<4xf32>", "%0 = tforge.relu %a : tensor<4xf32> -> tensor<4xf64>",
     "'tforge.relu' op result must have f32 elements, but has element type 'f64'"),
    ("%a: tensor<4x8xf32>, %b: tensor<4x7xf32>",
     "%0 = tforge.add %a, %b : tensor<4x8xf32>, tensor<4x7xf32> -> tensor<4x8xf32>",
     "'tforge.add' op operand shapes must match (no implicit broadcasting): lhs is 4x8, rhs is 4x7"),
    ("%a: tensor<4x8xf32>, %b: tensor<8xf32>", "%0 = tforge.add %a, %b : tensor<4x8xf32>, tensor<8xf32> -> tensor<4x8xf32>",
     "'tforge.add' op operand shapes must match (no implicit broadcasting): lhs is 4x8, rhs is 8"),
    ("%a: tensor<4x8xf32>", "%0 = tforge.add %a, %a : tensor<4x8xf32>, tensor<4x8xf32> -> tensor<8x4xf32>",
     "'tforge.add' op result shape 8x4 does not match operand shape 4x8"),
    ("%a: tensor<4x8xf32>", "%0 = tforge.relu %a : tensor<4x8xf32> -> tensor<4x9xf32>",
     "'tforge.relu' op result shape 4x9 does not match input shape 4x8"),
    ("%a: tensor<2x4x8xf32>, %b: tensor<8x4xf32>",
     "%0 = tforge.matmul %a, %b : tensor<2x4x8xf32>, tensor<8x4xf32> -> tensor<4x4xf32>",
     "'tforge.matmul' op lhs must be rank 2 (M x K), but has rank 3"),
    ("%a: tensor<4x8xf32>, %b: tensor<8xf32>", "%0 = tforge.matmul %a, %b : tensor<4x8xf32>, tensor<8xf32> -> tensor<4xf32>",
     "'tforge.matmul' op rhs must be rank 2 (K x N), but has rank 1"),
    ("%a: tensor<64x32xf32>, %b: tensor<16x16xf32>",
     "%0 = tforge.matmul %a, %b : tensor<64x32xf32>, tensor<16x16xf32> -> tensor<64x16xf32>",
     "'tforge.matmul' op contracting dimensions do not match: lhs is 64x32 (K = 32), rhs is 16x16 (K = 16)"),
    ("%a: tensor<64x32xf32>, %b: tensor<32x16xf32>",
     "%0 = tforge.matmul %a, %b : tensor<64x32xf32>, tensor<32x16xf32> -> tensor<16x64xf32>",
     "'tforge.matmul' op result shape must be 64x16 (M x N), but got 16x64"),
    ("%a: tensor<4x8xf32>, %b: tensor<1x8xf32>",
     "%0 = tforge.bias_add %a, %b : tensor<4x8xf32>, tensor<1x8xf32> -> tensor<4x8xf32>",
     "'tforge.bias_add' op bias must be rank 1, but has rank 2"),
    ("%a: tensor<4x8xf32>, %b: tensor<4xf32>",
     "%0 = tforge.bias_add %a, %b : tensor<4x8xf32>, tensor<4xf32> -> tensor<4x8xf32>",
     "'tforge.bias_add' op bias length 4 does not match the last dimension of input 4x8 (8)"),
    ("%a: tensor<f32>, %b: tensor<1xf32>", "%0 = tforge.bias_add %a, %b : tensor<f32>, tensor<1xf32> -> tensor<f32>",
     "'tforge.bias_add' op input must have rank >= 1, but is a scalar"),
    ("%a: tensor<4x8xf32>, %b: tensor<8xf32>",
     "%0 = tforge.bias_add %a, %b : tensor<4x8xf32>, tensor<8xf32> -> tensor<4x7xf32>",
     "'tforge.bias_add' op result shape 4x7 does not match input shape 4x8"),
]


@pytest.mark.parametrize("args,line,msg", INVALID)
def test_verifier_diagnostics(args, line, msg):
    prog = f"func.func @f({args}) {{\n  // a comment\n  {line}\n  return\n}}\n"
    err = compile_err(prog)
    col = 3 + line.index("=") + 2  # the op name follows "%0 = "
    assert err == f"t.mlir:3:{col}: error: {msg}", err


def test_example_program_plans_one_fused_launch():
    prog = ("// relu(x @ w + b)\nfunc.func @entry(%x: tensor<256x128xf32>, %w: tensor<128x256xf32>, "
            "%b: tensor<256xf32>) -> tensor<256x256xf32> {\n"
            "  %mm = tforge.matmul %x, %w : tensor<256x128xf32>, tensor<128x256xf32> -> tensor<256x256xf32>\n"
            "  %ba = tforge.bias_add %mm, %b : tensor<256x256xf32>, tensor<256xf32> -> tensor<256x256xf32>\n"
            "  %r = tforge.relu %ba : tensor<256x256xf32> -> tensor<256x256xf32>\n"
            "  return %r : tensor<256x256xf32>\n}\n")
    k = _lib.Kernel(prog, "")
    (l,) = k.launches()
    assert l["ops"] == "matmul+bias_add+relu" and l["family"] == "direct"
    assert [b["shape"] for b in k.buffers()] == [(256, 128), (128, 256), (1, 256), (256, 256)]


def test_module_wrapper_and_generic_form():
    prog = ("module {\n func.func @entry(%a: tensor<4x8xf32>) -> tensor<4x8xf32> {\n"
            '  %0 = "tforge.relu"(%a) : (tensor<4x8xf32>) -> tensor<4x8xf32>\n'
            "  return %0 : tensor<4x8xf32>\n }\n}\n")
    assert _lib.Kernel(prog).launches()[0]["family"] == "elementwise"


def test_gen_mlir_matches_reference_input():
    assert tc.gen_mlir("mbr", 2048, 2048, 2048) == (GOLDEN / "stage8_input_mbr_2048.mlir").read_text()


def test_naive_geometry_gpu_pipeline_lit():
    # test/Pipelines/gpu-pipeline.mlir: 67x33 @ 33x17, 16x16 blocks, 1x1 -> grid [2,5,1], block [16,16,1]
    k = _lib.Kernel(tc.gen_mlir("mbr", 67, 17, 33), "block-tile=16,16 thread-tile=1,1")
    l = k.launches()[0]
    assert l["grid"] == [2, 5, 1] and l["block"] == [16, 16, 1]


def test_default_options_are_naive_16x16():
    l = _lib.Kernel(tc.gen_mlir("mbr", 1024, 1024, 1024), "").launches()[0]
    want = json.loads((GOLDEN / "stage7_launch_mbr_1024.json").read_text())
    assert l["grid"] == want["grid"] and l["block"] == want["block"]


def test_staged_geometry_matches_reference_launch():
    want = json.loads((GOLDEN / "stage8_launch_mbr_2048.json").read_text())
    k = _lib.Kernel(tc.gen_mlir("mbr", 2048, 2048, 2048),
                    "block-tile=128,64 thread-tile=8,4 tile-k=16 promote=1 vectorize=1")
    l = k.launches()[0]
    assert l["grid"] == want["grid"] and l["block"] == want["block"]
    assert l["args"] == want["args"]  # result first, then A, B, bias
    assert l["family"] == "staged" and l["kernel"] == "tf_staged_b128x64_t8x4_k16"


def test_block_dims_gpu_tile_script_lit():
    # test/Transforms/gpu-tile-script.mlir:17: 32x64 / 2x4 -> block_dims [16, 16, 1]
    l = _lib.Kernel(tc.gen_mlir("mbr", 128, 256, 64), "block-tile=32,64 thread-tile=2,4").launches()[0]
    assert l["block"] == [16, 16, 1] and l["grid"] == [4, 4, 1]


def test_notpadded_located_error():
    # test/Pipelines/gpu-staged.mlir:39 -- N = 128 with BN = 48
    prog = tc.gen_mlir("mbr", 128, 128, 64)
    err = compile_err(prog, "block-tile=64,48 thread-tile=4,4 tile-k=16 promote=1")
    line = prog.splitlines().index(next(l for l in prog.splitlines() if "tforge.matmul" in l)) + 1
    col = prog.splitlines()[line - 1].index("tforge.matmul") + 1
    assert err == (f"t.mlir:{line}:{col}: error: tforge-gpu-tile: tile-k needs static tiles; pad the problem to "
                   "multiples of the block and K tiles")


def test_dimension_limits():
    """A dimension past int64 is a located "invalid dimension" (MLIR's type
    parser message); one past 2^31 - 1 parses but the kernels take 32-bit M, N
    and K, so planning refuses it at the op; 2^31 - 1 itself is accepted."""
    prog = tc.gen_mlir("relu", 4, 8).replace("4x8", "99999999999999999999x8", 1)
    line = next(i for i, l in enumerate(prog.splitlines(), 1) if "99999999999999999999" in l)
    col = prog.splitlines()[line - 1].index("99999999999999999999") + 1
    assert compile_err(prog) == f"t.mlir:{line}:{col}: error: invalid dimension"
    big = tc.gen_mlir("mbr", 2147483648, 16, 8)
    line = next(i for i, l in enumerate(big.splitlines(), 1) if "tforge.matmul" in l)
    col = big.splitlines()[line - 1].index("tforge.matmul") + 1
    assert compile_err(big) == (f"t.mlir:{line}:{col}: error: tforge-gpu-pipeline: dimensions above 2^31 - 1 are "
                                "not supported (M = 2147483648, N = 16, K = 8)")
    assert "dimensions above" in compile_err(tc.gen_mlir("matmul", 4, 4, 1 << 40))
    assert "dimensions above" in compile_err(tc.gen_mlir("relu", 1 << 31, 4))
    # rank-3 element op: the leading dimensions flatten to M = 2^33 (no overflow on the way)
    rank3 = tc.gen_mlir("relu", 4, 8).replace("4x8", "65536x131072x8")
    assert "dimensions above" in compile_err(rank3)
    huge3 = tc.gen_mlir("relu", 4, 8).replace("4x8", "9223372036854775807x9223372036854775807x8")
    assert "dimensions above" in compile_err(huge3)
    assert _lib.Kernel(tc.gen_mlir("mbr", 2147483647, 16, 8), "").launches()[0]["grid"] == [1, 134217728, 1]


def test_tile_k_needs_a_matmul():
    err = compile_err(tc.gen_mlir("relu", 64, 64), "tile-k=16")
    assert err.endswith("error: tforge-gpu-tile: tile-k needs a matmul")


@pytest.mark.parametrize("opts", ["block-tile=16,16,16", "thread-tile=3,1", "block-tile=16", "block-tile=0,16",
                                  "thread-tile=0,1"])
def test_tile_list_errors(opts):
    assert compile_err(tc.gen_mlir("mbr", 64, 64, 64), opts) == (
        "tforge-gpu-pipeline: block-tile and thread-tile need 2 values each, block a multiple of thread")


@pytest.mark.parametrize("opts,needle", [("bogus=1", "no such option bogus"), ("promote=maybe", "invalid value"),
                                         ("tile-k=x", "invalid value")])
def test_option_errors(opts, needle):
    assert needle in compile_err(tc.gen_mlir("mbr", 64, 64, 64), opts)


def test_relu_of_relu_folds_into_one_epilogue_op():
    """ReluOp::fold (lib/Dialect/TForge/TForgeFolders.cpp): relu is idempotent,
    so a fused relu after relu adds no operation."""
    t = "tensor<64x64xf32>"
    prog = (f"func.func @entry(%a: {t}, %b: {t}) -> {t} {{\n"
            f"  %0 = tforge.matmul %a, %b : {t}, {t} -> {t}\n"
            f"  %1 = tforge.relu %0 : {t} -> {t}\n"
            f"  %2 = tforge.relu %1 : {t} -> {t}\n"
            f"  %3 = tforge.relu %2 : {t} -> {t}\n"
            f"  return %3 : {t}\n}}\n")
    (l,) = _lib.Kernel(prog).launches()
    assert l["ops"] == "matmul+relu"


def test_split_k_geometry_and_errors():
    """split-k=S (a backend option) puts S workgroups per output tile on grid z."""
    staged = "block-tile=64,64 thread-tile=4,4 tile-k=32 promote=1 vectorize=1"
    l = _lib.Kernel(tc.gen_mlir("mbr", 64, 4096, 4096), staged + " split-k=8").launches()[0]
    assert l["grid"] == [64, 1, 8] and l["block"] == [16, 16, 1]
    assert _lib.Kernel(tc.gen_mlir("mbr", 64, 4096, 4096), staged).launches()[0]["grid"] == [64, 1, 1]
    prog = tc.gen_mlir("mbr", 64, 64, 256)  # 8 slabs of 32
    assert _lib.Kernel(prog, staged + " split-k=8").launches()[0]["grid"][2] == 8
    assert compile_err(prog, staged + " split-k=9").endswith(
        "error: tforge-gpu-pipeline: split-k 9 exceeds the 8 K slabs of this matmul")
    assert compile_err(prog, "split-k=2").endswith("error: tforge-gpu-pipeline: split-k needs tile-k")
    for bad in ("split-k=0", "split-k=65", "split-k=x"):
        assert "invalid value" in compile_err(prog, staged + " " + bad)
    # unfused program: split-k applies to the matmul launch; bias_add and relu run as they are
    unf = _lib.Kernel(tc.gen_mlir("mbr", 128, 128, 256), staged + " split-k=4 fuse-elementwise=0").launches()
    assert [(l["ops"], l["grid"][2]) for l in unf] == [("matmul", 4), ("bias_add", 1), ("relu", 1)]


def test_mask_edges_accepts_any_shape():
    """mask-edges=1 (a backend option) lifts the NOTPADDED rule: the grid
    covers the shape with ceil-divided tiles and the kernel masks edges."""
    staged = "block-tile=128,64 thread-tile=8,4 tile-k=16 promote=1 vectorize=1"
    prog = tc.gen_mlir("mbr", 777, 1111, 333)
    assert "tile-k needs static tiles" in compile_err(prog, staged)
    l = _lib.Kernel(prog, staged + " mask-edges=1").launches()[0]
    assert l["grid"] == [18, 7, 1] and (l["m"], l["n"], l["k"]) == (777, 1111, 333)
    assert _lib.Kernel(prog, staged + " mask-edges=1 split-k=3").launches()[0]["grid"] == [18, 7, 3]
    assert "mask-edges needs promote=1" in compile_err(prog, staged.replace("promote=1", "promote=0") + " mask-edges")
    # multiples of the tiles need no masks, so promote=0 is fine there
    _lib.Kernel(tc.gen_mlir("mbr", 256, 128, 64), staged.replace("promote=1", "promote=0") + " mask-edges=1")
    assert tg.padded_shape(777, 1111, 333, staged + " mask-edges=1") == (777, 1111, 333)
    assert tg.padded_shape(777, 1111, 333, "{" + staged + " mask-edges}") == (777, 1111, 333)


def test_options_accept_braces_bools_and_print_script(capfd):
    k = _lib.Kernel(tc.gen_mlir("mbr", 256, 256, 64),
                    "{block-tile=128,128 thread-tile=8,8 tile-k=32 promote=true vectorize=1 print-script=1}")
    err = capfd.readouterr().err
    assert "tf_staged_b128x128_t8x8_k32" in err and "matmul+bias_add+relu" in err
    assert k.launches()[0]["lds_bytes"] == 2 * (128 * 36 + 32 * 136) * 4 + 128 * 4


def test_staged_config_without_waves_is_rejected():
    """A block that is not a whole number of 64-lane waves and has no stand-in
    wave layout (BM, BN not multiples of 8) is refused with the reason."""
    err = compile_err(tc.gen_mlir("mbr", 72, 72, 64), "block-tile=36,36 thread-tile=6,6 tile-k=8 promote=1 vectorize=1")
    assert "not a whole number of 64-lane waves" in err


def test_sub_wave_config_runs_on_one_wave():
    """The reference's 32-thread block-tile=32,32 thread-tile=8,4 runs one
    64-lane wave over the whole 32x32 block, and reports that block."""
    k = _lib.Kernel(tc.gen_mlir("mbr", 64, 64, 64), "block-tile=32,32 thread-tile=8,4 tile-k=8 promote=1 vectorize=1")
    launch = k.launches()[0]
    assert launch["kernel"] == "tf_staged_b32x32_t4x4_k8"
    assert launch["block"] == [8, 8, 1] and launch["grid"] == [2, 2, 1]


def test_unfused_program_has_three_launches():
    k = _lib.Kernel(tc.gen_mlir("mbr", 64, 64, 64), "fuse-elementwise=0")
    assert [l["ops"] for l in k.launches()] == ["matmul", "bias_add", "relu"]
    assert [l["family"] for l in k.launches()] == ["direct", "elementwise", "elementwise"]


def test_residual_block_two_launches():
    k = _lib.Kernel(tc.gen_mlir("resmlp", 256, 128, 512),
                    "block-tile=128,128 thread-tile=8,8 tile-k=32 promote=1 vectorize=1")
    l1, l2 = k.launches()
    assert l1["ops"] == "matmul+bias_add+relu" and (l1["m"], l1["n"], l1["k"]) == (256, 512, 128)
    assert l2["ops"] == "matmul+bias_add+relu+add" and (l2["m"], l2["n"], l2["k"]) == (256, 128, 512)
    assert l1["args"][0].startswith("tmp") and l2["args"][1] == l1["args"][0]  # h stays on the device
    assert l2["args"][-1] == "arg0"  # the residual add reads x


def test_self_add_and_multi_use_values():
    t = "tensor<64x64xf32>"
    prog = (f"func.func @entry(%a: {t}, %b: {t}) -> {t} {{\n"
            f"  %0 = tforge.matmul %a, %b : {t}, {t} -> {t}\n"
            f"  %1 = tforge.relu %0 : {t} -> {t}\n"
            f"  %2 = tforge.add %1, %1 : {t}, {t} -> {t}\n"
            f"  return %2 : {t}\n}}\n")
    (l,) = _lib.Kernel(prog).launches()
    assert l["ops"] == "matmul+relu+add"
    # a matmul result used twice cannot be updated in place: it is materialised
    prog2 = (f"func.func @entry(%a: {t}, %b: {t}) -> {t} {{\n"
             f"  %0 = tforge.matmul %a, %b : {t}, {t} -> {t}\n"
             f"  %1 = tforge.relu %0 : {t} -> {t}\n"
             f"  %2 = tforge.add %1, %0 : {t}, {t} -> {t}\n"
             f"  return %2 : {t}\n}}\n")
    assert [l["ops"] for l in _lib.Kernel(prog2).launches()] == ["matmul", "relu+add"]


@pytest.mark.parametrize("bad,needle", [
    ("func.func @entry(%a: tensor<4xf32>) -> tensor<4xf32> {\n  %0 = tforge.relu %b : tensor<4xf32> -> tensor<4xf32>\n"
     "  return %0 : tensor<4xf32>\n}\n", "use of undeclared SSA value name '%b'"),
    ("func.func @entry(%a: tensor<4xf32>) -> tensor<4xf32> {\n  %0 = tforge.relu %a : tensor<4xf32> -> tensor<4xf32>\n}\n",
     "must end with 'return'"),
    ("func.func @entry(%a: tensor<4xf32>) -> tensor<4xf32> {\n  %0 = tforge.mul %a : tensor<4xf32> -> tensor<4xf32>\n",
     "unknown operation 'tforge.mul'"),
    ("func.func @entry(%a: tensor<4xf32>) -> tensor<4xf32> {\n  %0 = tforge.relu %a : tensor<4xf32> -> tensor<4xf32>\n"
     "  return %a : tensor<4xf32>\n}\n", "returning an argument"),
])
def test_structural_errors(bad, needle):
    assert needle in compile_err(bad)
