"""The C ABI's host code under AddressSanitizer (a debug build of the library with only the host
pass instrumented; the device code is the same).  The reference has no sanitizer runs (it is
single-threaded host code); this checks that every entry point's argument validation and error
reporting stays inside its memory, on inputs the checks must reject: null pointers, negative,
unit and huge extents.  CPU only: the probe hands every pointer argument a host buffer, which must
not reach a GPU, so it is skipped where one is visible."""
import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

from aneforge_amd import _build

ROOT = Path(__file__).resolve().parents[1]
OK_CALLS = {"afx_abi_version", "afx_moe_route_sync_words"}          # no arguments to check
OK_NULL = {"afx_graph_destroy", "afx_event_destroy"}                 # NULL handle: nothing to destroy


def _asan_lib() -> Path:
    srcs = list(_build.CSRC.glob("*.hip")) + list(_build.CSRC.glob("*.h"))
    out = _build.OUT_ASAN
    if not out.is_file() or out.stat().st_mtime < max(s.stat().st_mtime for s in srcs):
        _build.build(sanitize=True)
    return out


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="passes host buffers as device pointers; CPU-only probe")
def test_c_abi_host_paths_under_address_sanitizer():
    rt = _build.asan_runtime()
    if not rt or not os.path.isfile(rt):
        pytest.skip("no AddressSanitizer runtime in this toolchain")
    lib = _asan_lib()
    env = dict(os.environ, AFX_LIB=str(lib), LD_PRELOAD=rt, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               HIP_VISIBLE_DEVICES="")
    r = subprocess.run([sys.executable, str(ROOT / "tests" / "asan_probe.py"), str(ROOT / "aneforge_amd" / "_hip.py")],
                       env=env, capture_output=True, text=True, timeout=600)
    assert "ERROR: AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0, r.stderr[-4000:]
    res = json.loads(r.stdout.strip().splitlines()[-1])
    calls = [k for k in res if not k.startswith("ws:")]
    assert len(calls) >= 4 * 50, len(calls)
    for key in calls:
        mode, name = key.split(":", 1)
        rc, msg = res[key]
        if name in OK_CALLS or (mode == "zero" and name in OK_NULL):
            assert rc >= 0, (key, rc, msg)
        else:
            assert rc < 0 and msg, (key, rc, msg)   # rejected, with a message
    ws = {int(k[len("ws:afx_sample_ws_bytes("):-1]): v[0] for k, v in res.items() if k.startswith("ws:")}
    assert ws[-5] == -1 and ws[0] == -1 and ws[(1 << 21) + 1] == -1
    assert 0 < ws[1] < ws[2048] < ws[2049] < ws[151936] < ws[1 << 21]
