"""Interleaved A/B timing of builds of libhymt_hip.so: the harness behind the
variant measurements (a kernel changed in one source file, timed against the
library as built, on one box, in alternating runs so that clock drift and
box-to-box spread weigh on every build alike).

    python -m hymt2sharp_amd.ab build DIR [--flags "-DNAME=1 ..."]
        DIR/libhymt_hip.so from the package's sources, each DIR/<name>.hip or
        DIR/<name>.cpp replacing the package's file of that name (compiled
        with the package's flags for that file, plus --flags, with csrc/ on
        the include path); the package's other objects (_build/, from
        build.build_hip) are linked as they are.

    python -m hymt2sharp_amd.ab run --leg prefill --key prefill.roofline.avg_us \\
            [--key ...] [--rounds 3] DIR [DIR ...]
        runs `bench.py --no-cpu --no-spread --only LEG` once per build per
        round -- the package's own library first, then each DIR's (through
        HYMT_HIP_LIB) -- and prints the values at the dotted key paths of
        each run's JSON line, then their median per build.

Keys name the bench line's fields, e.g. `prefill.roofline.avg_us` (config 3's
flash kernel), `prefill.ms_per_call`, `config4.ms_per_call`,
`roofline.call.avg_us` (config 2's decode call),
`config5.by_context.32768.kernels.decode_attn.avg_us`,
`gemm.shapes.o_m2048.mfma_plan_us`, `model.prefill.ms`, `model.tokens_per_s`.
"""
from __future__ import annotations

import argparse
import json
import os
import shutil
import statistics
import subprocess
import sys

from . import build as B

SOURCES = tuple(B.HIP_SOURCES)


def build_variant(d: str, flags: str = "") -> str:
    """DIR/libhymt_hip.so with DIR's replacement sources; returns its path."""
    d = os.path.abspath(d)
    own = [s for s in SOURCES if os.path.isfile(os.path.join(d, s))]
    if not own:
        raise SystemExit(f"{d} holds none of the library's sources ({', '.join(SOURCES)})")
    objs = []
    for src in SOURCES:
        stem = os.path.splitext(src)[0]
        if src in own:
            obj = os.path.join(d, stem + ".o")
            B._run([B.HIPCC, *B.HIP_FLAGS, *B.HIP_SOURCES[src], *flags.split(), "-I", B.CSRC, "-c",
                    os.path.join(d, src), "-o", obj])
        else:
            obj = os.path.join(B.BUILD_DIR, stem + ".o")
            if not os.path.isfile(obj):
                raise SystemExit(f"{obj} missing: build the package first (python -m hymt2sharp_amd.build)")
        objs.append(obj)
    lib = os.path.join(d, "libhymt_hip.so")
    B._run([B.HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-L/opt/rocm/lib", "-lhipblaslt",
            "-Wl,-rpath,/opt/rocm/lib", "-o", lib + ".tmp"])
    os.replace(lib + ".tmp", lib)
    for src in own:
        os.remove(os.path.join(d, os.path.splitext(src)[0] + ".o"))
    return lib


def value_at(doc: dict, key: str):
    """The value at a dotted path of the bench line (None if absent)."""
    v = doc
    for part in key.split("."):
        if not isinstance(v, dict) or part not in v:
            return None
        v = v[part]
    return v


def bench_line(text: str) -> dict:
    lines = [ln for ln in text.splitlines() if ln.startswith("{")]
    if not lines:
        raise RuntimeError("no JSON line in the bench output")
    return json.loads(lines[-1])


def run_ab(leg: str, keys: list[str], dirs: list[str], rounds: int = 3, timeout: int = 300) -> dict:
    """{build: {key: [value per round]}}, the package's library as 'base'."""
    builds = [("base", B.HIP_LIB)] + [(os.path.basename(os.path.normpath(d)) or d,
                                        os.path.join(os.path.abspath(d), "libhymt_hip.so")) for d in dirs]
    for name, lib in builds:
        if not os.path.isfile(lib):
            raise SystemExit(f"{name}: {lib} is not built")
    res = {name: {k: [] for k in keys} for name, _ in builds}
    cmd = [sys.executable, os.path.join(B.ROOT, "bench.py"), "--no-cpu", "--no-spread", "--only", leg]
    for r in range(rounds):
        for name, lib in builds:
            env = dict(os.environ, HYMT_HIP_LIB=lib)
            p = subprocess.run(cmd, env=env, cwd=B.ROOT, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                               text=True, timeout=timeout)
            if p.returncode != 0:
                sys.stdout.write(p.stdout[-4000:])
                raise SystemExit(f"{name}: bench.py exited with {p.returncode}")
            doc = bench_line(p.stdout)
            vals = {k: value_at(doc, k) for k in keys}
            for k, v in vals.items():
                res[name][k].append(v)
            print(f"round {r} {name:12s} " + " ".join(f"{k}={v}" for k, v in vals.items()), flush=True)
    return res


def summary(res: dict) -> str:
    out = []
    for name, by_key in res.items():
        cells = []
        for k, vs in by_key.items():
            nums = [v for v in vs if isinstance(v, (int, float))]
            cells.append(f"{k}={statistics.median(nums):.4g}" if nums else f"{k}=n/a")
        out.append(f"median {name:12s} " + " ".join(cells))
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m hymt2sharp_amd.ab")
    sub = ap.add_subparsers(dest="cmd", required=True)
    b = sub.add_parser("build", help="build a variant library")
    b.add_argument("dir")
    b.add_argument("--flags", default="", help="extra hipcc flags for the replaced sources")
    r = sub.add_parser("run", help="interleaved bench runs of the package's library and the variants")
    r.add_argument("dirs", nargs="*")
    r.add_argument("--leg", required=True)
    r.add_argument("--key", action="append", required=True)
    r.add_argument("--rounds", type=int, default=3)
    r.add_argument("--timeout", type=int, default=300, help="seconds per bench run")
    a = ap.parse_args(argv)
    if a.cmd == "build":
        print(build_variant(a.dir, a.flags))
    else:
        print(summary(run_ab(a.leg, a.key, a.dirs, a.rounds, a.timeout)))


if __name__ == "__main__":
    if shutil.which(B.HIPCC) is None and not os.path.isfile(B.HIPCC):
        raise SystemExit(f"{B.HIPCC} not found")
    main()
