"""The kernels that use matrix cores (chunk_prep, chunk_scan, chunk_wide,
chunk_bwd), compiled for gfx950 with the library's own flags: along every
control-flow path of every kernel, no instruction reads a v_mfma result
fewer wait states after the product than hipcc itself places within one
block for that product (8 for the 16x16x32 and 16x16x16 fp16 / bf16 forms, 10
for 16x16x4 fp32; an s_nop N counts N + 1, any other instruction 1). Results
in VGPRs (v) and in accumulation registers (a, read back by v_accvgpr_read or
as MFMA operands) are both followed.

hipcc (ROCm 7.2) has emitted reads two to five wait states after a product
issued inside a branch, when the read follows the join: the read then sees
stale result registers (the narrow scan's last output tile of fp32 inputs
came out with every fourth row wrong). The kernels are written so that no
branch separates a product from its first reads; this test keeps it so."""
import os
import re
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

import pytest

from pseudobrain_amd import build

SOURCES = ("chunk_prep.hip", "chunk_scan.hip", "chunk_wide.hip", "chunk_bwd.hip")
NEED = {"v_mfma_f32_16x16x32_f16": 8, "v_mfma_f32_16x16x32_bf16": 8, "v_mfma_f32_16x16x16_f16": 8,
        "v_mfma_f32_16x16x16_bf16": 8, "v_mfma_f32_16x16x4_f32": 10}
_REG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")
_STORES = ("ds_write", "ds_add", "global_store", "buffer_store", "global_atomic", "buffer_atomic", "flat_store")


def vgprs(text):
    """The vector registers an operand text names, as ('v', n) or ('a', n)."""
    out = set()
    for m in _REG.finditer(text):
        if m.group(5) is not None:
            out.add((m.group(4), int(m.group(5))))
        else:
            out.update((m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1))
    return out


def reads(ins):
    """VGPRs an instruction reads (an MFMA's accumulator input excepted: a
    chain of products into one accumulator has its own, shorter rule)."""
    op, _, rest = ins.partition(" ")
    args = [a.strip() for a in rest.split(",")] if rest else []
    if op.startswith("v_mfma"):
        return vgprs(",".join(args[1:3]))
    if op.startswith(_STORES):
        return vgprs(rest)
    if op.startswith(("v_", "ds_", "global_", "buffer_", "flat_")):
        return vgprs(",".join(args[1:]))
    return set()


def functions(asm):
    """(name, [instruction text], {label: instruction index}) per kernel."""
    out = []
    for line in asm.split("\n"):
        m = re.match(r"^(_Z\S*):", line)
        if m:
            out.append((m.group(1), [], {}))
            continue
        if not out:
            continue
        text = line.split(";")[0].strip()
        if not text:
            continue
        lab = re.match(r"^(\.?[\w$.]+):$", text)
        if lab:
            out[-1][2][lab.group(1)] = len(out[-1][1])
        elif not text.startswith("."):
            out[-1][1].append(text)
    return out


def short_reads(asm):
    """(kernel, product, reader, wait states) for every read of a product's
    result closer than NEED along some path."""
    found = []
    for name, ins, labels in functions(asm):
        def successors(k):
            op, _, rest = ins[k].partition(" ")
            if op in ("s_endpgm", "s_setpc_b64", "s_trap"):
                return []
            if op == "s_branch":
                return [labels[rest.split()[0]]]
            if op.startswith("s_cbranch"):
                return [k + 1, labels[rest.split()[0]]]
            return [k + 1]

        for k, text in enumerate(ins):
            op = text.split()[0]
            if not op.startswith("v_mfma"):
                continue
            need = NEED.get(op)
            assert need is not None, f"no wait-state rule for {op}"
            dst = vgprs(text.split(None, 1)[1].split(",")[0])
            stack, seen = [(s, 0) for s in successors(k)], set()
            while stack:
                j, w = stack.pop()
                if j >= len(ins) or (j, w) in seen:
                    continue
                seen.add((j, w))
                if reads(ins[j]) & dst:
                    found.append((name, text, ins[j], w))
                    continue
                opj, _, rest = ins[j].partition(" ")
                if opj.startswith("v_mfma") and vgprs(rest.split(",")[0]) >= dst:
                    continue  # the result is overwritten before any read
                w2 = w + (int(rest.split()[0], 0) + 1 if opj == "s_nop" else 1)
                if w2 < need:
                    stack.extend((s, w2) for s in successors(j))
    return found


def test_checker_finds_a_read_after_a_join():
    """A read two wait states behind a product issued in a branch is found;
    the straight-line form with eight is not."""
    bad = """_Zk:
	v_mfma_f32_16x16x32_f16 v[8:11], v[0:3], v[4:7], v[8:11]
	s_cbranch_scc1 .LBB0_2
	v_mfma_f32_16x16x32_f16 v[8:11], v[0:3], v[4:7], v[8:11]
.LBB0_2:
	s_nop 0
	v_mul_f32_e32 v12, v11, v13
	s_endpgm
"""
    hits = short_reads(bad)
    assert len(hits) == 2 and {h[3] for h in hits} == {1, 2}
    good = bad.replace("s_nop 0", "s_nop 7")
    assert short_reads(good) == []


def test_checker_follows_accumulation_registers():
    """A product into accumulation registers, read back by v_accvgpr_read after
    a join, is found as well; a product into other registers is not."""
    bad = """_Zk:
	v_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[4:7], a[0:3]
	s_cbranch_scc1 .LBB0_2
	v_mov_b32_e32 v9, v8
.LBB0_2:
	v_accvgpr_read_b32 v12, a3
	s_endpgm
"""
    hits = short_reads(bad)
    assert {h[3] for h in hits} == {1, 2} and all("v_accvgpr_read" in h[2] for h in hits)
    assert short_reads(bad.replace("a[0:3], v[0:3]", "a[4:7], v[0:3]")) == []
    assert vgprs("a[2:3], v5") == {("a", 2), ("a", 3), ("v", 5)}


def test_no_mfma_result_is_read_early():
    cc = build.hipcc()
    if not os.path.exists(cc) and cc == "hipcc":
        pytest.skip("hipcc is not installed")
    with tempfile.TemporaryDirectory() as tmp:
        def compile_one(src):
            out = os.path.join(tmp, src.replace(".hip", ".s"))
            subprocess.run([cc, *build.HIPCC_FLAGS, f"-I{build.INCLUDE}", "--cuda-device-only", "-S",
                            os.path.join(build.CSRC, src), "-o", out], check=True, capture_output=True)
            with open(out) as f:
                return src, f.read()

        with ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
            listings = list(pool.map(compile_one, SOURCES))
    problems = []
    for src, asm in listings:
        assert "v_mfma" in asm, src
        problems += [f"{src}: {name[-48:]}: '{prod}' read by '{rd}' after {w}"
                     for name, prod, rd, w in short_reads(asm)]
    assert not problems, "\n".join(problems[:20])
