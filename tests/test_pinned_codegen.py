"""The hand-ordered ("pinned") main loop of the large LDS tiles, checked on the gfx950 code this
build compiles (CPU only: hipcc -S, no GPU).

On these tiles the weight widening (v_perm for e5m2, v_cvt_scalef32_pk_f16_fp8 for e4m3fn) and
the MFMAs are inline asm, so the compiler's hazard tracking does not see them and the source
keeps the ordering rules itself. This test checks them in the compiled loops:
  * every MFMA accumulates in place (destination = accumulator source), and no other vector
    instruction in a loop body reads or writes an accumulator register (a compiler copy of an
    accumulator between MFMAs would read an unfinished result);
  * a widened weight register is written at least one MFMA before the MFMA that reads it (a
    register an MFMA has read as its A or B operand may be overwritten right after it: the
    compiler's own code for builtin MFMAs does that, e.g. in the split-K tiles);
  * after the last loop, three `s_nop 7` come before any non-MFMA instruction reads an MFMA's
    result (the epilogue's scaling, the LoRA term)."""

import re
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO))

# the pinned tiles: default schedule (5th template argument 1), wave tiles of at least 64 x 64
PINNED = r"scaled_mm_lds_kernelILi(256ELi256ELi4ELi2|256ELi128ELi4ELi2|128ELi256ELi2ELi4|128ELi128ELi2ELi2|" \
         r"256ELi192ELi4ELi2|128ELi384ELi2ELi4)ELi1E"


@pytest.fixture(scope="module")
def bodies(tmp_path_factory):
    import __graft_entry__

    b = __graft_entry__.load_build_module()
    out = tmp_path_factory.mktemp("asm") / "scaled_mm_lds.s"
    cmd = [b._hipcc(), *b.HIP_FLAGS, "--cuda-device-only", "-S", str(b.CSRC / "scaled_mm_lds.hip"), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stderr[-2000:]
    found = {}
    name = None
    for line in out.read_text().splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            name = m.group(1) if re.search(PINNED, m.group(1)) else None
            if name:
                found[name] = []
            continue
        if name is None:
            continue
        if line.startswith(".Lfunc_end"):
            name = None
            continue
        found[name].append(line)
    return found


def _regs(op: str) -> set:
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", op)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", op)
    return {int(m.group(1))} if m else set()


def _instr(line: str):
    s = line.split(";")[0].strip()
    if not s or s.endswith(":") or s.startswith("."):
        return None
    parts = s.split(None, 1)
    ops = [o.strip() for o in parts[1].split(",")] if len(parts) > 1 else []
    ops = [o.split()[0] if o else o for o in ops]
    return parts[0], ops


def _loop_accumulators(body: list) -> set:
    """Destination registers of the MFMAs inside the loops (the main loop's accumulators; the LoRA
    epilogue's MFMAs after the loop may reuse other registers)."""
    accs = set()
    for a, b in _loops(body):
        for line in body[a:b]:
            ins = _instr(line)
            if ins and ins[0].startswith("v_mfma"):
                accs |= _regs(ins[1][0])
    return accs


def _loops(body: list) -> list:
    """(start, end) line ranges of the loops: a 'Loop Header' label to its last back edge."""
    out = []
    for i, line in enumerate(body):
        if "Loop Header" in line:
            label = line.split(":")[0]
            ends = [j for j, l in enumerate(body) if "s_cbranch" in l and l.split(";")[0].strip().endswith(label)]
            if ends:
                out.append((i, max(ends)))
    return out


def test_pinned_tiles_are_compiled(bodies):
    # 4 output/weight-format variants x (no LoRA + 2 LoRA kinds for e5m2) per tile; at least the six tiles
    assert len({re.search(PINNED, n).group(1) for n in bodies}) == 6, sorted(bodies)[:3]


def test_mfmas_in_place_and_accumulators_untouched_in_loops(bodies):
    for name, body in bodies.items():
        accs = _loop_accumulators(body)
        loops = _loops(body)
        assert loops and accs, name
        for a, b in loops:
            for line in body[a:b]:
                ins = _instr(line)
                if not ins or not ins[0].startswith("v_"):
                    continue
                op, ops = ins
                if op.startswith("v_mfma"):
                    assert ops[0] == ops[3], f"{name}: MFMA not in place: {line.strip()}"
                    continue
                touched = set().union(*[_regs(o) for o in ops]) if ops else set()
                assert not (touched & accs), f"{name}: loop instruction touches an accumulator: {line.strip()}"


def test_widened_weights_written_one_mfma_before_use(bodies):
    for name, body in bodies.items():
        for a, b in _loops(body):
            seq = [x for x in (_instr(l) for l in body[a:b]) if x]
            n_mfma = 0
            last_write = {}  # register -> MFMA count when a widening instruction wrote it
            checked = 0
            for op, ops in seq:
                if op in ("v_perm_b32", "v_cvt_scalef32_pk_f16_fp8"):
                    for r in _regs(ops[0]):
                        last_write[r] = n_mfma
                elif op.startswith("v_mfma"):
                    for r in _regs(ops[1]):  # the weights are the first source operand
                        if r in last_write:
                            assert n_mfma - last_write[r] >= 1, f"{name}: v{r} read by the next MFMA after widening"
                            checked += 1
                    n_mfma += 1
            assert checked > 0, f"{name}: no widened operand found in a loop"


def test_wait_states_before_accumulators_are_read(bodies):
    """Between the last loop and the pad, no other vector instruction reads a register whose latest
    write (in program order; the loop's accumulators count as written by MFMAs) was an MFMA. The
    stages after the last full round of the ring run there, outside any loop, with their own
    MFMAs; a register the compiler re-initialises with an ordinary move first (the accumulators'
    zero on the path that skips the loop) is not an MFMA result."""
    for name, body in bodies.items():
        loops = _loops(body)
        end = max(b for _, b in loops)
        pads = [i for i in range(end, len(body) - 2)
                if all("s_nop 7" in body[i + k] for k in range(3))]
        assert pads, f"{name}: no wait-state pad after the main loop"
        from_mfma = set(_loop_accumulators(body))
        for line in body[end:pads[0]]:
            ins = _instr(line)
            if not ins or not ins[0].startswith("v_"):
                continue
            op, ops = ins
            dst = _regs(ops[0]) if ops else set()
            if op.startswith("v_mfma"):
                from_mfma |= dst
                continue
            src = set().union(*[_regs(o) for o in ops[1:]]) if len(ops) > 1 else set()
            assert not (src & from_mfma), f"{name}: MFMA result read before the wait states: {line.strip()}"
            from_mfma -= dst
