"""Code-generation guards for the hot kernels (CPU only: compiles to gfx950 assembly).

Each check pins a property the kernels' speed depends on and that a small source change
can silently lose:
  * GEMV kernels read their problem descriptors with scalar loads: no flat (per-lane)
    loads, and no readfirstlane "waterfall" loops (a loop of v_readfirstlane + 64-bit
    compares that makes a per-lane buffer resource uniform, once per chunk);
  * no register spills (scratch) in the GEMV kernels (a spill of a value just loaded
    makes the wave wait for that load, serialising the prologue's loads);
  * the GEMV expands weights with masks only and reads its activations for the dot
    products with scalar loads;
  * the GEMM's main loop is free of scratch traffic and of waterfall loops;
  * no lane read (v_readfirstlane / v_readlane) is written as inline asm: the compiler
    inserts no wait states before an asm statement that reads a VGPR its previous VALU
    instruction wrote, and such a read can return the stale value (it did, for the GEMV's
    chunk bounds, with wrong sums as the result);
  * the cross-workgroup hand-offs that run without a fence (the split-K parts' int32
    tiles, the decode q/k/v outputs polled by the attention workgroups) keep their
    device-coherent stores and loads and the wait before the arrival count.
"""
import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "rotor-rag_amd" / "csrc"
sys.path.insert(0, str(CSRC))
from build import DEVICE_FLAGS  # noqa: E402  (the library's own device flags)

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "--cuda-device-only", "-S", *DEVICE_FLAGS]


def _asm(src, tmp_path):
    if not Path(HIPCC).exists():
        pytest.skip("hipcc not available")
    out = tmp_path / (Path(src).stem + ".s")
    r = subprocess.run([HIPCC, *FLAGS, str(CSRC / src), "-o", str(out)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text()


def _kernels(asm):
    """kernel symbol -> its instruction text (label to the function's end, every block);
    "__meta__" -> {symbol: its .amdhsa_kernel descriptor block}."""
    out, name, body = {}, None, []
    for line in asm.splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            name, body = m.group(1), []
            continue
        if name is not None:
            if line.startswith(".Lfunc_end"):
                out[name] = "\n".join(body)
                name = None
            else:
                body.append(line)
    out["__meta__"] = {m.group(1): m.group(2)
                       for m in re.finditer(r"\.amdhsa_kernel (\S+)\n(.*?)\.end_amdhsa_kernel", asm, re.S)}
    return out


def _waterfalls(text):
    return len(re.findall(r"v_readfirstlane_b32[^\n]*\n\s*v_readfirstlane_b32[^\n]*\n(?:[^\n]*\n){0,2}\s*v_cmp_eq_u64", text))


@pytest.fixture(scope="module")
def gemv(tmp_path_factory):
    return _kernels(_asm("rt_gemv.hip", tmp_path_factory.mktemp("gemv")))


@pytest.fixture(scope="module")
def gemm(tmp_path_factory):
    return _kernels(_asm("rt_gemm.hip", tmp_path_factory.mktemp("gemm")))


def test_gemv_kernels_scalar_descriptors_no_spills(gemv):
    names = [n for n in gemv if "gemv_rows_kernel" in n or "gemv_ksplit_kernel" in n]
    assert len(names) >= 9, names
    for n in names:
        t = gemv[n]
        assert "flat_load" not in t, f"{n}: per-lane flat loads"
        assert _waterfalls(t) == 0, f"{n}: readfirstlane loop"
        assert "scratch_" not in t, f"{n}: register spills"


def test_gemv_prologue_source_preloaded(gemv):
    # the KSPLIT kernels get their row source (x, aux, aux2, K, mode, eps: 9 dwords), the
    # inline problem count, nw and its reciprocal in SGPRs at wave launch
    for n in [n for n in gemv if "gemv_ksplit_kernel" in n]:
        m = re.search(r"\.amdhsa_user_sgpr_kernarg_preload_length\s+(\d+)", gemv["__meta__"][n])
        assert m and int(m.group(1)) >= 12, n


def test_no_inline_asm_lane_reads(gemv, gemm):
    for kernels in (gemv, gemm):
        for n, t in kernels.items():
            if n == "__meta__":
                continue
            for block in re.findall(r";;#ASMSTART(.*?);;#ASMEND", t, re.S):
                assert "v_readfirstlane" not in block and "v_readlane" not in block, f"{n}: inline-asm lane read"


def test_gemv_rows_reads_activations_with_scalar_loads(gemv):
    (n,) = [n for n in gemv if "gemv_rows_kernelILi1ELi0E" in n]
    t = gemv[n]
    assert "s_load_dwordx16" in t or "s_load_dwordx8" in t
    # the only per-lane activation loads are the 16-byte ones of the sum-x pass (one
    # round of 4 per token), issued before the weight loop (the epilogue's per-row scale
    # and residual loads come after it)
    loads = re.findall(r"global_load\w*", t[: t.index("buffer_load_dwordx4")])
    assert loads and set(loads) == {"global_load_dwordx4"} and len(loads) <= 4, loads


def test_gemv_decodes_with_masks_only(gemv):
    # device code g = w + 1: the chunk loop expands weights by shifts and masks (no
    # v_perm lookup table) and reduces sum x with DPP adds
    for n in [n for n in gemv if "gemv_rows_kernel" in n or "gemv_ksplit_kernel" in n]:
        t = gemv[n]
        assert "0x1ff00" not in t, n  # the lookup operand of the former v_perm decode
        assert "0xc0c0c0c" in t and "0x3030303" in t, n
        assert "row_bcast:31" in t, n


def test_gemm_main_loop_clean(gemm):
    tiles = [n for n in gemm if "gemm_kernel" in n]
    splitk = [n for n in gemm if "gemm_splitk_kernel" in n]
    assert len(tiles) >= 3 and len(splitk) >= 1, list(gemm)
    for n in tiles + splitk:
        t = gemm[n]
        assert _waterfalls(t) == 0, f"{n}: readfirstlane loop"
        assert "v_mfma_i32_32x32x32_i8" in t
        assert "global_load_lds_dwordx4" in t  # operands reach LDS by direct loads
    for n in tiles:
        # spills may only appear in the epilogue (after the first output store)
        body = gemm[n].split("buffer_store_dword")[0]
        assert "scratch_load" not in body, f"{n}: scratch reloads before the epilogue"
    for n in splitk:
        assert "scratch_" not in gemm[n], f"{n}: register spills"


def test_splitk_uses_no_static_lds(gemm):
    # two split-K workgroups (4 waves x 4 stages x 5 KiB = 80 KiB each) share a CU's 160 KiB of
    # LDS only if the kernel declares no static LDS on top (4 bytes halved the residency and
    # slowed a 7-projection launch from 12.7 to 15.5 us)
    for n in [n for n in gemm if "gemm_splitk_kernel" in n]:
        m = re.search(r"\.amdhsa_group_segment_fixed_size\s+(\d+)", gemm["__meta__"][n])
        assert m and int(m.group(1)) == 0, n


def test_splitk_exchange_is_coherent(gemm):
    # The split-K parts hand their int32 tiles to the last arriver without a fence: the
    # tiles are stored device-coherent (sc1), every store has completed (s_waitcnt
    # vmcnt(0)) and the workgroup has passed a barrier before the arrival count is added
    # to, and the last arriver reads the other parts' tiles device-coherent.  A compiler
    # that dropped the coherence bits or moved the wait would break the exchange silently.
    for n in [n for n in gemm if "gemm_splitk_kernel" in n]:
        t = gemm[n]
        i = t.index("global_atomic_add")
        before, after = t[:i], t[i:]
        stores = re.findall(r"global_store_dword\b[^\n]*", before)
        assert stores and all(re.search(r"\bsc1\b", s) for s in stores), f"{n}: tile stores {stores}"
        tail = before[before.rindex("global_store_dword"):]
        assert re.search(r"s_waitcnt vmcnt\(0\)(.|\n)*s_barrier", tail), f"{n}: no wait + barrier before the count"
        # the last arriver's reads of the other parts' tiles: from the count to its reset
        # (a device-coherent store of zero); the epilogue's scale loads follow
        reset = re.search(r"global_store_dword\b[^\n]*\bsc1\b", after)
        assert reset, f"{n}: no device-coherent reset of the arrival count"
        loads = re.findall(r"global_load_dword\b[^\n]*", after[:reset.start()])
        assert loads and all(re.search(r"\bsc1\b", s) for s in loads), f"{n}: tile loads {loads}"


def test_attention_handoff_is_coherent(gemv):
    # The q/k/v GEMV of the decode step stores its outputs as 64-bit (epoch, value) words
    # device-coherent (sc1) and the attention workgroups of the same launch poll them with
    # device-coherent loads (between s_sleep); the epoch is read coherent too.
    names = [n for n in gemv if "gemv_ksplit_kernel" in n and "AttnTail" in n]
    assert len(names) >= 3, names
    for n in names:
        t = gemv[n]
        lines = t.splitlines()
        sleeps = [i for i, l in enumerate(lines) if "s_sleep" in l]
        polls = [l for i in sleeps for l in lines[i + 1:i + 9] if "global_load_dwordx2" in l]
        assert polls and all(re.search(r"\bsc1\b", l) for l in polls), f"{n}: polls {polls}"
        tagged = [l for l in re.findall(r"global_store_dwordx2[^\n]*", t) if re.search(r"\bsc1\b", l)]
        assert tagged, f"{n}: no device-coherent 64-bit store of the tagged outputs"
        assert re.search(r"global_load_dword\b[^\n]*\bsc1\b", t), f"{n}: the epoch is not read coherent"
