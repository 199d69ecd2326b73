"""Host-side sanitizer run of the C ABI's descriptor validation (CPU only, no GPU call).

Every library source is compiled with AddressSanitizer and UndefinedBehaviorSanitizer on its host code
(`-Xarch_host`; the device code is built as usual and never launched) and linked with
`tests/sanitize/validate_fuzz.cpp`. That driver sends edge-value and seeded random descriptors through
`ssd_validate`, `ssd_workspace_bytes` and the shape checks of `ssd_materialize_L` / `ssd_decay_chunk`
(with null tensors, so nothing launches); any signed overflow, out-of-bounds access or invalid load aborts
the run. The build is cached in the temp directory under a hash of its inputs: the first run compiles for
about two minutes on eight cores, later runs only execute it.
"""
import hashlib
import os
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "dhammic-ai_amd" / "csrc"
DRIVER = ROOT / "tests" / "sanitize" / "validate_fuzz.cpp"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-std=c++17", "-O1", "-g", "-fPIC", f"-I{ROOT / 'include'}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=all",
]


def _inputs():
    files = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.h")) + sorted((ROOT / "include").glob("*.h")) + [DRIVER]
    h = hashlib.sha256(" ".join(FLAGS).encode())
    for f in files:
        h.update(f.name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(map(str, cmd))}\n{r.stdout[-4000:]}")


def _build():
    out = Path(tempfile.gettempdir()) / f"ssd_sanitize_{_inputs()}"
    exe = out / "validate_fuzz"
    if exe.exists():
        return exe
    out.mkdir(parents=True, exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    objs = [out / (s.stem + ".o") for s in srcs]
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        list(ex.map(lambda so: _run([HIPCC, *FLAGS, "-c", str(so[0]), "-o", str(so[1])]), zip(srcs, objs)))
    drv = out / "validate_fuzz.o"
    _run([HIPCC, *FLAGS, "-x", "c++", "-c", str(DRIVER), "-o", str(drv)])
    tmp = out / "validate_fuzz.tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
          *map(str, objs), str(drv), "-o", str(tmp)])
    os.replace(tmp, exe)
    return exe


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")
def test_validation_under_sanitizers():
    exe = _build()
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stdout[-4000:]
    assert "validate_fuzz: ok" in r.stdout
