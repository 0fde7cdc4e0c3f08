"""The kernels under the debug build (libpbgdn_debug.so, -DPBGDN_DEBUG): every
kernel fills its LDS with NaN before its first use, and every entry point
fills its outputs and workspaces with NaN (0xff bytes) before it launches.
A kernel that reads LDS its own launch has not written, an element of an
output that no kernel writes, or a workspace record the scan reads before the
prep kernel writes it then shows as NaN, and the parity checks of the cases
below (each one a test of another file, run again through the debug library,
against the same oracle and tolerances) fail. In-place buffers (state pools,
carried conv tails) keep their contents: they hold inputs. The debug build
also counts the barriers each wave of the narrow scan passes (its loader and
compute waves run separate loops meant to have the same barrier sequence)
and every workgroup's waves must agree."""
import contextlib
import ctypes

import numpy as np
import pytest
import torch

from pseudobrain_amd import _lib
from pseudobrain_amd import gated_deltanet as gd
from pseudobrain_amd.workloads import generate
from tests import (test_gpu_backward, test_gpu_chunk, test_gpu_chunk_k256, test_gpu_chunk_layer, test_gpu_decode_layer,
                   test_gpu_fla_schema, test_gpu_layer, test_gpu_prologue_varlen, test_gpu_recurrent,
                   test_gpu_state_pools, test_gpu_wide)

pytestmark = pytest.mark.gpu

CASES = {
    # prefill: the narrow scan (one sequence, chained packed sequences), padding, fp32 inputs (range
    # scale, Tb's low part), fp16 inputs, the wide scan, state slots
    "narrow scan, Qwen3-Next heads, T=4096": lambda: test_gpu_chunk.test_prefill_qwen3next_shape(4096),
    "narrow scan, T=65 (a padded chunk)": lambda: test_gpu_chunk.test_padding_and_short_sequences(65),
    "float32 inputs, T=2048": test_gpu_chunk.test_prefill_small_fp32_inputs,
    "float16 inputs": lambda: test_gpu_chunk.test_input_dtypes_and_zero_state(torch.float16),
    "chained narrow scan, 8 packed sequences": test_gpu_chunk.test_varlen_small,
    "chained narrow scan, 300 short sequences": lambda: test_gpu_chunk.test_many_short_sequences(300, 2, 4, 64),
    "wide scan, B=4 T=300": lambda: test_gpu_wide.test_wide_batch(4, 300, 16, 32, torch.bfloat16),
    "wide scan, packed ragged": test_gpu_wide.test_wide_packed_sequences_with_empty_and_ragged_lengths,
    "prefill state slots, bf16 pool": lambda: test_gpu_state_pools.test_prefill_state_slots(torch.bfloat16),
    # 256-wide keys: key halves (two tiles a workgroup), one wave a tile (four tiles), packed sequences
    "256-wide keys, T=300 V=256": lambda: test_gpu_chunk_k256.test_lengths_and_value_widths(300, 256),
    "256-wide keys, 4-tile workgroups": test_gpu_chunk_k256.test_four_wave_workgroups,
    "256-wide keys, packed sequences": test_gpu_chunk_k256.test_packed_sequences,
    # prefill with the layer epilogue: fused in the wide scan, and the two-kernel path
    "fused layer epilogue": lambda: test_gpu_chunk_layer.test_fused_in_the_wide_scan(
        4, 300, 16, torch.bfloat16, torch.float32),
    "narrow scan, then the layer epilogue": lambda: test_gpu_chunk_layer.test_narrow_scan_then_epilogue(
        1, 1000, torch.bfloat16, torch.float32),
    "chained narrow scan, then the layer epilogue": lambda: test_gpu_chunk_layer.test_two_pass_shapes(
        1, 700, 128, None),
    # decode
    "decode step, B=64": test_gpu_recurrent.test_decode_b64_one_step,
    "multi-token recurrent, bf16": lambda: test_gpu_recurrent.test_sequential_kernel_multi_token(
        128, 128, torch.bfloat16),
    "speculative verify": test_gpu_recurrent.test_speculative_verify_keeps_the_state_after_every_token,
    "decode step, bf16 state slots": lambda: test_gpu_state_pools.test_decode_16bit_state_slots(torch.bfloat16),
    "fused decode layer step, B=64": test_gpu_decode_layer.test_decode_step_qwen3next_b64,
    # the layer prologue and epilogue
    "prologue, Qwen3-Next shape": lambda: test_gpu_layer.test_prologue_qwen3next_shape("max"),
    "prologue, short inputs": lambda: test_gpu_layer.test_prologue_short_inputs_keep_part_of_the_tail(2),
    "packed prologue, serving batch": test_gpu_prologue_varlen.test_varlen_qwen3next_serving_batch,
    "epilogue": lambda: test_gpu_layer.test_epilogue(128, torch.bfloat16, torch.bfloat16, torch.float32),
    # backward
    "backward, bf16 GQA 1 -> 4": lambda: test_gpu_backward.test_backward_matches_the_oracle(
        1, 333, 1, 4, 128, 64, torch.bfloat16),
    "backward, float32, 16 chunks": lambda: test_gpu_backward.test_backward_matches_the_oracle(
        1, 1000, 2, 2, 128, 128, torch.float32),
    # fla's residuals (gc, A) of the reference's op
    "chunk residuals, GQA 2 -> 4": lambda: test_gpu_fla_schema.test_residuals_match_the_oracle(
        1, 130, 2, 4, 64, torch.bfloat16),
}


AUDIT_ROWS, AUDIT_WAVES = 4096, 12  # chunk_scan.hip's debug barrier audit


def scan_barrier_rows(lib, reset=False):
    """The narrow scan's per-wave barrier counts, [AUDIT_ROWS, 12] (a row per
    workgroup of the last launch that used it; 0xffffffff where none did)."""
    fn = lib.pbgdn_debug_scan_barriers
    fn.argtypes, fn.restype = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int], ctypes.c_int
    out = np.zeros((AUDIT_ROWS, AUDIT_WAVES), dtype=np.uint32)
    assert fn(out.ctypes.data, AUDIT_ROWS, int(reset)) == _lib.OK
    return out


@pytest.mark.parametrize("name", list(CASES))
def test_case_under_the_debug_build(name):
    """The case's own parity checks pass with the kernels' LDS and the outputs
    poisoned, and every workgroup of the narrow scan had its loader and
    compute waves pass the same number of barriers."""
    print(f"[debug build] {name}", flush=True)
    with _lib.debug_library() as lib:
        scan_barrier_rows(lib, reset=True)
        CASES[name]()
        torch.cuda.synchronize()
        rows = scan_barrier_rows(lib)
    used = rows[:, 0] != 0xffffffff
    mismatched = np.nonzero((rows != rows[:, :1]).any(axis=1))[0]
    print(f"[debug build] {name}: narrow-scan workgroups audited {int(used.sum())}, "
          f"barriers per wave {sorted(set(rows[used, 0].tolist()))[:4]}", flush=True)
    assert mismatched.size == 0, f"waves of workgroup rows {mismatched[:8].tolist()} passed different barrier counts"


def test_debug_build_poisons_unwritten_outputs():
    """Positive control: with cu_seqlens ending before T the rows past the last
    packed sequence belong to no sequence and no kernel writes them. The normal
    build leaves what the caller put there; the debug build leaves NaN."""
    q, k, v, g, beta, h0 = generate(1, 128, 2, 4, 128, 64, torch.bfloat16, 0.02, seed=3, nstates=1)
    cu = torch.tensor([0, 64], dtype=torch.int32, device="cuda")
    for debug in (False, True):
        out = torch.full((1, 128, 4, 64), 7.0, dtype=torch.bfloat16, device="cuda")
        with _lib.debug_library() if debug else contextlib.nullcontext():
            with torch.no_grad():
                gd.chunk_fwd(*(x.cuda() for x in (q, k, v, g, beta)), 128 ** -0.5, h0.cuda(), cu, out=out)
            torch.cuda.synchronize()
        assert torch.isfinite(out[:, :64]).all(), debug
        tail = out[:, 64:]
        assert bool(torch.isnan(tail).all()) if debug else bool((tail == 7.0).all()), debug
