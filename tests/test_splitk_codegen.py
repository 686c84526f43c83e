"""The K-split arrival protocol of the small-M kernel, the split-K LDS tiles and the LoRA
down-projection, checked on the gfx950 code this build compiles (CPU only: hipcc -S, no GPU).

Each split writes its fp32 partial with device-coherent (sc1) stores, waits for them to be
acknowledged (vmcnt(0)) and crosses a workgroup barrier before one thread's returning atomic add
on the tile's arrival counter; that thread waits for the atomic's result (vmcnt(0)) before
writing the last-arrival flag to LDS, and the partial loads (sc1) of the last arrival come after
the barrier that publishes the flag. Relaxed agent-scope atomics carry no ordering of their own:
this order in the compiled code is what the protocol rests on, so a compiler or source change
that breaks it fails here."""

import re
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO))


def _asm(tmp_path, src: str) -> str:
    import __graft_entry__

    b = __graft_entry__.load_build_module()
    out = tmp_path / (Path(src).stem + ".s")
    cmd = [b._hipcc(), *b.HIP_FLAGS, "--cuda-device-only", "-S", str(b.CSRC / src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text()


def _bodies(asm: str, kernel_re: str) -> dict:
    """Instruction lines (comments stripped) of every function whose symbol matches kernel_re."""
    out = {}
    lines = asm.splitlines()
    i = 0
    while i < len(lines):
        m = re.match(r"^(_Z\S+):", lines[i])
        if m and re.search(kernel_re, m.group(1)):
            body = []
            i += 1
            while i < len(lines) and not lines[i].startswith(".Lfunc_end"):
                s = lines[i].split(";")[0].strip()
                if s:
                    body.append(s)
                i += 1
            out[m.group(1)] = body
        i += 1
    return out


def _is_vmcnt0(s: str) -> bool:
    return s.startswith("s_waitcnt") and "vmcnt(0)" in s


def _check_protocol(name: str, body: list) -> None:
    atomics = [i for i, s in enumerate(body) if re.match(r"global_atomic_add\S*\s", s) and re.search(r"\bsc0\b", s)]
    assert len(atomics) == 1, f"{name}: expected one returning arrival atomic, found {len(atomics)}"
    a = atomics[0]

    def is_part_store(s):
        return re.match(r"(global|buffer)_store\S*\s", s) and re.search(r"\bsc1\b", s)

    def is_part_load(s):
        return re.match(r"(global|buffer)_load\S*\s", s) and re.search(r"\bsc1\b", s)

    stores = [i for i in range(a) if is_part_store(body[i])]
    assert stores, f"{name}: no device-coherent partial stores before the arrival atomic"
    between = body[stores[-1] + 1:a]
    w = next((k for k, s in enumerate(between) if _is_vmcnt0(s)), None)
    assert w is not None, f"{name}: partial stores not waited for (vmcnt(0)) before the arrival atomic"
    assert "s_barrier" in between[w + 1:], f"{name}: no barrier between the partials' wait and the atomic"
    after = body[a + 1:]
    ds = next((k for k, s in enumerate(after) if s.startswith("ds_write")), None)
    assert ds is not None, f"{name}: the atomic's result is not published through LDS"
    assert any(_is_vmcnt0(s) for s in after[:ds]), f"{name}: the flag is written before the atomic's result returned"
    bar = next((k for k in range(ds + 1, len(after)) if after[k] == "s_barrier"), None)
    assert bar is not None, f"{name}: no barrier after the flag write"
    loads = [k for k, s in enumerate(after) if is_part_load(s)]
    assert loads, f"{name}: no device-coherent partial loads after the atomic"
    assert min(loads) > bar, f"{name}: a partial load is issued before the barrier that publishes the flag"
    assert not [i for i in range(a) if is_part_load(body[i])], \
        f"{name}: a device-coherent partial load precedes the arrival atomic"


@pytest.mark.parametrize("src,kernel_re,min_kernels", [
    ("scaled_mm_smallm.hip", r"scaled_mm_smallm_kernel", 8),
    ("lora_down.hip", r"lora_down_kernel", 4),
    ("scaled_mm_lds.hip", r"scaled_mm_lds_kernelILi(64ELi64|64ELi128|32ELi128)E", 12),
])
def test_split_k_arrival_order_in_compiled_code(tmp_path, src, kernel_re, min_kernels):
    bodies = _bodies(_asm(tmp_path, src), kernel_re)
    assert len(bodies) >= min_kernels, f"{src}: found {len(bodies)} kernels matching {kernel_re}"
    for name, body in bodies.items():
        _check_protocol(name, body)


_GOOD = ["buffer_store_dwordx4 v[0:3], v2, s[12:15], 0 offen sc1", "s_waitcnt vmcnt(0)", "s_barrier",
         "global_atomic_add v2, v2, v3, s[30:31] sc0", "s_waitcnt vmcnt(0)", "ds_write_b32 v2, v0", "s_barrier",
         "ds_read_b32 v2, v0", "buffer_load_dwordx4 v[4:7], v2, s[12:15], 0 offen sc1",
         "global_store_dword v8, v8, s[0:1] sc1"]


@pytest.mark.parametrize("mutate", ["none", "no_store_wait", "no_store_barrier", "no_result_wait",
                                    "load_before_barrier", "load_before_atomic", "nonreturning_atomic"])
def test_protocol_checker_rejects_broken_orders(mutate):
    """The checker above on hand-made instruction sequences: the protocol's order passes, and
    each way of breaking it is caught."""
    body = list(_GOOD)
    if mutate == "no_store_wait":
        body.pop(1)
    elif mutate == "no_store_barrier":
        body.pop(2)
    elif mutate == "no_result_wait":
        body.pop(4)
    elif mutate == "load_before_barrier":
        body.insert(6, body.pop(8))
    elif mutate == "load_before_atomic":
        body.insert(3, body.pop(8))
    elif mutate == "nonreturning_atomic":
        body[3] = "global_atomic_add v2, v3, s[30:31]"
    if mutate == "none":
        _check_protocol("good", body)
    else:
        with pytest.raises(AssertionError):
            _check_protocol(mutate, body)


def test_one_pass_quantize_barrier_order_in_compiled_code(tmp_path):
    """quant_resident_kernel's grid barrier: each workgroup's partial maximum
    is stored device-coherently (sc1) and acknowledged (vmcnt(0)) before its
    returning arrival atomic; the partials are read (sc1 loads) only after the
    wait loop has ended and a workgroup barrier has published its outcome."""
    bodies = _bodies(_asm(tmp_path, "quant_prepack.hip"), r"quant_resident_kernel")
    assert len(bodies) >= 2, f"found {len(bodies)} one-pass quantize kernels"
    for name, body in bodies.items():
        atomics = [i for i, s in enumerate(body) if re.match(r"global_atomic_add\S*\s", s)]
        assert atomics, f"{name}: no arrival atomic"
        a = atomics[0]
        assert re.search(r"\bsc0\b", body[a]), f"{name}: the first arrival atomic does not return its result"
        stores = [i for i in range(a) if re.match(r"global_store\S*\s", body[i]) and re.search(r"\bsc1\b", body[i])]
        assert stores, f"{name}: no device-coherent partial store before the arrival"
        assert any(_is_vmcnt0(s) for s in body[stores[-1] + 1:a]), f"{name}: the partial is not acknowledged first"
        sleeps = [i for i in range(a, len(body)) if body[i].startswith("s_sleep")]
        assert sleeps, f"{name}: no wait loop after the arrival"
        bar = next((k for k in range(sleeps[-1], len(body)) if body[k] == "s_barrier"), None)
        assert bar is not None, f"{name}: no barrier after the wait loop"
        after = [k for k in range(bar, len(body)) if re.match(r"global_load\S*\s", body[k]) and re.search(r"\bsc1\b", body[k])]
        assert after, f"{name}: no device-coherent partial loads after the barrier"
