"""CPU: the split-K ticket protocol checked in the gfx950 assembly hipcc emits.

The kernels that merge partial results of several workgroups inside one launch
(the decode, the prefill and the split-K projections) rely on what the ISA
does, not on the C++ memory model: partials written with device-coherent
(`sc1`) stores, `s_waitcnt vmcnt(0)` before the ticket, the ticket an RMW atomic
returning its old value, merge loads device-coherent, and no whole-L2 write-back
or invalidate.  A toolchain that emitted other code for the `sc1` buffer
builtins, the relaxed agent-scope atomics or the inline wait would break the
merges silently on the GPU; this test makes it fail here instead.

Rules, for every kernel holding a ticket (`*_atomic_add ... sc0`):
  1. no `buffer_wbl2` / `buffer_inv`;
  2. walking back from each ticket in program order, `s_waitcnt vmcnt(0)` comes
     before any vector-memory store;
  3. every `buffer_store*` carries `sc1` (partials and their LSEs are written
     with the buffer-store builtins; outputs and page writes use global stores);
  4. every `buffer_load*` after the first ticket in program order carries `sc1`,
     except LDS-DMA (`lds`) and non-temporal (`nt`) page loads;
  5. the ticket is reset with a device-coherent dword store (`sc1`).
Each rule is also shown to catch a mistake planted in a copy of the decode
source: the wait removed, the partial stores' `sc1` removed, the merge loads'
`sc1` removed.
"""
from __future__ import annotations

import re
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from flexengine_amd import build as B

if shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists():
    pytest.skip("hipcc is not installed", allow_module_level=True)

# source file -> kernel families that take tickets (each must be found)
FILES = {
    "paged_decode.hip": ("piece_decode_kernel", "balanced_decode_kernel"),
    "prefill.hip": ("prefill_dma_kernel", "prefill_kernel"),
    "gemm_fused.hip": ("gemm_fused_kernel",),
    "gemm_rows64.hip": ("gemm_rows64_kernel",),
}

_STORE = re.compile(r"^\s*(buffer|global)_store\w*")
_BSTORE = re.compile(r"^\s*buffer_store\w*")
_BLOAD = re.compile(r"^\s*buffer_load\w*")
_TICKET = re.compile(r"^\s*(global|buffer)_atomic_add\w*\s.*\bsc0\b")
_WAIT0 = re.compile(r"^\s*s_waitcnt\s+vmcnt\(0\)")


def _assemble(src: Path, out: Path, include: Path) -> Path:
    flags = [f for f in B.HIP_FLAGS if f != "-fPIC"]
    cmd = [B.hipcc(), *flags, "-I", str(B.INCLUDE_DIR), "-I", str(include),
           "--cuda-device-only", "-S", str(src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out


def _functions(path: Path):
    name, body = None, []
    for line in path.read_text().splitlines():
        m = re.match(r"^(_Z\w+):", line)
        if m:
            name, body = m.group(1), []
            continue
        if name and line.startswith(".Lfunc_end"):
            yield name, body
            name = None
            continue
        if name:
            body.append(line.split(";")[0].rstrip())   # drop comments


def violations(path: Path) -> tuple[dict[str, int], list[tuple[str, str]]]:
    """(ticket kernels found per name, [(kernel, broken rule)])."""
    found: dict[str, int] = {}
    bad: list[tuple[str, str]] = []
    for name, body in _functions(path):
        tickets = [i for i, l in enumerate(body) if _TICKET.match(l)]
        if not tickets:
            continue
        found[name] = len(tickets)
        if any(re.match(r"^\s*buffer_(wbl2|inv)", l) for l in body):
            bad.append((name, "1: whole-L2 write-back / invalidate"))
        for i in tickets:
            j = i - 1
            while j >= 0 and not _STORE.match(body[j]) and not _WAIT0.match(body[j]):
                j -= 1
            if j < 0 or _STORE.match(body[j]):
                bad.append((name, f"2: no vmcnt(0) between the last store and the ticket ({i})"))
        stores = [l for l in body if _BSTORE.match(l)]
        if not stores or any(not re.search(r"\bsc1\b", l) for l in stores):
            bad.append((name, "3: a buffer store without sc1"))
        loads = [l for l in body[tickets[0] + 1:]
                 if _BLOAD.match(l) and not re.search(r"\b(lds|nt)\b", l)]
        if not loads or any(not re.search(r"\bsc1\b", l) for l in loads):
            bad.append((name, "4: a merge buffer load without sc1"))
        if not any(re.match(r"^\s*global_store_dword\s.*\bsc1\b", l) for l in body):
            bad.append((name, "5: no sc1 dword store (ticket reset)"))
    return found, bad


@pytest.fixture(scope="module")
def assembled(tmp_path_factory):
    tmp = tmp_path_factory.mktemp("isa")
    with ThreadPoolExecutor(max_workers=len(FILES)) as pool:
        outs = list(pool.map(lambda f: _assemble(B.CSRC_DIR / f, tmp / (f + ".s"), B.CSRC_DIR),
                             FILES))
    return dict(zip(FILES, outs))


@pytest.mark.parametrize("src", list(FILES))
def test_ticket_kernels_follow_the_protocol(assembled, src):
    found, bad = violations(assembled[src])
    for family in FILES[src]:
        assert any(family in name for name in found), f"{family} has no ticket in {src}"
    assert not bad, "\n".join(f"{n}: {r}" for n, r in bad)


def _plant(text: str, start: str, end: str, old: str, new: str) -> str:
    i = text.index(start)
    j = text.index(end, i)
    seg = text[i:j]
    assert seg.count(old) >= 1, old
    return text[:i] + seg.replace(old, new) + text[j:]


PLANTS = {
    # the wave's wait for its partial stores before the ticket
    "no_wait": ("auto store_partial", "merge_pieces<D, E, PAD>(a, b, h",
                "wait_stores();  // this wave", "// (planted) no wait"),
    # the partial outputs written with default caching instead of sc1
    "store_not_coherent": ("auto store_partial", "store_coherent(a.ws_lse",
                           "0, kSc1);", "0, 0);"),
    # the merge reads the partials through the L2
    "load_not_coherent": ("void merge_pieces", "template <int D, class Core>",
                          "0, kSc1));", "0, 0));"),
}


@pytest.mark.parametrize("plant", list(PLANTS))
def test_planted_protocol_mistakes_are_caught(plant):
    start, end, old, new = PLANTS[plant]
    src = (B.CSRC_DIR / "paged_decode.hip").read_text()
    with tempfile.TemporaryDirectory(prefix="fe_isa_plant_") as tmp:
        tmp = Path(tmp)
        for h in B.CSRC_DIR.glob("*.h"):
            shutil.copy(h, tmp / h.name)
        (tmp / "planted.hip").write_text(_plant(src, start, end, old, new))
        found, bad = violations(_assemble(tmp / "planted.hip", tmp / "planted.s", tmp))
    hit = {n for n, _ in bad if "piece_decode_kernel" in n}
    piece = {n for n in found if "piece_decode_kernel" in n}
    assert piece and hit == piece, (plant, sorted(piece - hit))
