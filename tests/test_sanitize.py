"""The engine's parsers of untrusted bytes (GGUF files, exported
directories, config.json, GRWS1 state bytes) under AddressSanitizer and
UndefinedBehaviorSanitizer on the CPU.  The reference rejects bad or
truncated state files and checkpoints with an error
(crates/omg-wgpu/src/engine.rs:536-579, model.rs:66-254,742-795); here every
mutated input must be accepted or refused, and neither may read out of
bounds or hit undefined behaviour on the way: the harness
(tests/sanitize/parsers_main.cpp) is built with g++
-fsanitize=address,undefined from the same sources as the library and
aborts with the sanitizer's report on the first fault."""
from __future__ import annotations

import json
import os
import random
import shutil
import struct
import subprocess
from pathlib import Path

import pytest

import grande_amd as g
from tests.common import gemma4_tiny, gguf_tiny
from tests.gguf_writer import write_gemma3

HERE = Path(__file__).resolve().parent
CSRC = HERE.parent / "grande_amd" / "csrc"
BUILD = HERE / "sanitize" / "_build"
SOURCES = [CSRC / "model.cpp", CSRC / "gguf.cpp", CSRC / "state.cpp", HERE / "sanitize" / "parsers_main.cpp"]


@pytest.fixture(scope="module")
def harness() -> Path:
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    BUILD.mkdir(parents=True, exist_ok=True)
    exe = BUILD / "parsers_asan"
    deps = SOURCES + list(CSRC.glob("*.h"))
    if not exe.exists() or exe.stat().st_mtime < max(p.stat().st_mtime for p in deps):
        # built under a name of this process, then moved into place: parallel
        # test workers never run a half-written binary
        tmp = exe.with_name(f"{exe.name}.{os.getpid()}")
        cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
               "-fno-sanitize-recover=all", f"-I{CSRC}", *map(str, SOURCES), "-o", str(tmp)]
        subprocess.run(cmd, check=True)
        os.replace(tmp, exe)
    return exe


def run(exe: Path, args: list[str]) -> list[str]:
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    res = subprocess.run([str(exe), *args], capture_output=True, text=True, env=env, timeout=600)
    assert res.returncode == 0, f"sanitizer report:\n{res.stderr[-4000:]}"
    lines = res.stdout.splitlines()
    assert len(lines) == len(args)
    return lines


def mutate(raw: bytes, rnd: random.Random, span: int, cut: float) -> bytes:
    b = bytearray(raw)
    for _ in range(rnd.randint(1, 4)):
        pos = rnd.randrange(min(len(b), span))
        b[pos] = rnd.choice([0, 0xFF, 0x7F, 0x80, rnd.randrange(256)])
    if rnd.random() < cut:
        b = b[: rnd.randrange(len(b) + 1)]
    return bytes(b)


def test_gguf_mutations_under_sanitizers(harness, tmp_path):
    for ci, cfg in enumerate([gguf_tiny(), gemma4_tiny()]):
        w = g.Weights.synth(cfg, 3, g.Q8, g.Q4)
        src = tmp_path / f"src{ci}.gguf"
        write_gemma3(src, cfg, w)
        raw = src.read_bytes()
        rnd = random.Random(100 + ci)
        args = [f"gguf:{src}"]
        for i in range(120):
            p = tmp_path / f"m{ci}_{i}.gguf"
            p.write_bytes(mutate(raw, rnd, 8000, 0.2))
            args.append(f"gguf:{p}")
        lines = run(harness, args)
        assert lines[0].startswith("ok"), lines[0]
        assert any(line.startswith("refused") for line in lines[1:])


def test_state_bytes_mutations_under_sanitizers(harness, tmp_path):
    good = b"GRWS1\0" + struct.pack("<I", 1) + b"m" + struct.pack("<I", 3) + struct.pack("<III", 1, 2, 3)
    good += struct.pack("<I", 2)
    for layer in range(2):
        good += struct.pack("<III", layer, 0, 16) + bytes(range(16))
    rnd = random.Random(7)
    (tmp_path / "good.state").write_bytes(good)
    args = [f"state:{tmp_path / 'good.state'}"]
    for i in range(400):
        p = tmp_path / f"s{i}.state"
        p.write_bytes(mutate(good, rnd, len(good), 0.3))
        args.append(f"state:{p}")
    # lengths near 2^32 in every length field
    for off in (6, 11, 27, 31 + 4 * 2, 51):
        b = bytearray(good)
        b[off:off + 4] = struct.pack("<I", 0xFFFFFFF0)
        p = tmp_path / f"big{off}.state"
        p.write_bytes(bytes(b))
        args.append(f"state:{p}")
    lines = run(harness, args)
    assert lines[0].startswith("ok"), lines[0]
    assert sum(line.startswith("refused") for line in lines) > 100


def test_config_and_manifest_mutations_under_sanitizers(harness, tmp_path):
    cfg = gguf_tiny()
    w = g.Weights.synth(cfg, 5, g.Q4, g.Q8)
    g.export_dir(w, tmp_path / "model")
    conf = (tmp_path / "model" / "config.json").read_text()
    man = (tmp_path / "model" / "manifest.json").read_text()
    rnd = random.Random(9)
    args = [f"dir:{tmp_path / 'model'}", f"config:{tmp_path / 'model' / 'config.json'}"]
    odd = ["1e400", "-1", "18446744073709551616", "1.5", "\"x\"", "null", "[]", "{}", "-0", "4294967297",
           "99999999999999999999999"]
    for i in range(60):
        # numbers of every awkward kind into config.json and manifest.json fields
        c = json.loads(conf)
        key = rnd.choice(sorted(c))
        c[key] = json.loads(rnd.choice(odd))
        p = tmp_path / f"c{i}.json"
        p.write_text(json.dumps(c))
        args.append(f"config:{p}")
        d = tmp_path / f"d{i}"
        shutil.copytree(tmp_path / "model", d)
        m = json.loads(man)
        ent = rnd.choice(m["files"])
        fld = rnd.choice([k for k in ent if not isinstance(ent[k], (list, dict))] or ["name"])
        ent[fld] = json.loads(rnd.choice(odd))
        (d / "manifest.json").write_text(json.dumps(m))
        args.append(f"dir:{d}")
    for i in range(40):
        p = tmp_path / f"t{i}.json"
        p.write_bytes(mutate(conf.encode(), rnd, len(conf), 0.3))
        args.append(f"config:{p}")
    lines = run(harness, args)
    assert lines[0].startswith("ok") and lines[1].startswith("ok"), lines[:2]


def test_packing_under_sanitizers(harness, tmp_path):
    """pack_groups + align_groups on request shapes with empty prefixes,
    empty groups (also last) and branchless groups, at both alignments:
    every index the layout records stays inside it."""
    def req(groups, first=0, resident=False, align=32):
        return {"first": first, "resident": resident, "align": align, "rows": 1 << 20,
                "groups": [{"prefix": p, "branches": [{"tokens": t, "want": w} for t, w in bs]} for p, bs in groups]}

    shapes = [
        [([1, 2, 3, 4, 5], [([6, 7, 8], [2])]), ([1, 2, 3], []), ([], [])],  # empty last group
        [([], [([4, 5], [1])]), ([], []), ([9], [([3], [0])])],
        [([], []), ([1, 2], [([3], [0])])],
        [([7] * 40, [([1] * 33, [0, 32])]), ([], []), ([], [])],
    ]
    rnd = random.Random(21)
    for _ in range(60):
        gs = []
        for _ in range(rnd.randint(1, 5)):
            p = [rnd.randrange(100) for _ in range(rnd.choice([0, 0, 1, 3, 33, 70]))]
            bs = []
            for _ in range(rnd.choice([0, 1, 2, 3])):
                n = rnd.choice([1, 2, 17, 40])
                bs.append(([rnd.randrange(100) for _ in range(n)], sorted({rnd.randrange(n) for _ in range(2)})))
            gs.append((p, bs))
        shapes.append(gs)
    args = []
    for i, gs in enumerate(shapes):
        for align in (32, 64):
            for resident in (False, True):
                p = tmp_path / f"r{i}_{align}_{int(resident)}.json"
                p.write_text(json.dumps(req(gs, first=i % len(gs), resident=resident, align=align)))
                args.append(f"pack:{p}")
    lines = run(harness, args)
    # a request whose tokens are all empty is refused ("empty request"); the rest pack
    assert sum(line.startswith("ok") for line in lines) > len(lines) // 2
    assert all(line.startswith("ok") or "empty request" in line for line in lines), \
        [line for line in lines if not line.startswith("ok")][:3]
