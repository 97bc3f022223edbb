"""Child process of tests/test_asan_host.py (run with the ASan runtime preloaded and AFX_LIB naming
the host-ASan build): calls every int-returning entry point of the C ABI with null pointers, then
with a dummy host buffer for every pointer and each of -1, 1 and 2^30 for every integer, and prints
{"mode:name": [rc, message]} as JSON.  Without a GPU every call must end in an argument check or a
failed HIP call, returning a negative code with a message.  Loads aneforge_amd/_hip.py on its own
(ctypes only), so neither torch nor the package's other modules load under the sanitizer."""
import ctypes as C
import importlib.util
import json
import sys

spec = importlib.util.spec_from_file_location("afx_hip_standalone", sys.argv[1])
hip = importlib.util.module_from_spec(spec)
spec.loader.exec_module(hip)
lib = hip.load()
buf = (C.c_char * (1 << 20))()
dummy = C.cast(buf, C.c_void_p)
INTS = {"zero": 0, "neg": -1, "one": 1, "huge": 1 << 30}


def args_for(types, mode):
    out = []
    for t in types:
        if t in (C.c_int, C.c_longlong):
            out.append(INTS[mode])
        elif t in (C.c_float, C.c_double):
            out.append(float(INTS[mode]))
        else:
            out.append(None if mode == "zero" else C.cast(dummy, t))
    return out


res = {}
for mode in INTS:
    for name, (rt, types) in hip.SIGNATURES.items():
        if rt is not C.c_int:
            continue
        rc = getattr(lib, name)(*args_for(types, mode))
        res[f"{mode}:{name}"] = [int(rc), hip.last_error() if rc < 0 else ""]
for V in (-5, 0, 1, 2048, 2049, 151936, 1 << 21, (1 << 21) + 1):      # workspace sizes over their ranges
    res[f"ws:afx_sample_ws_bytes({V})"] = [int(lib.afx_sample_ws_bytes(V)), ""]
print(json.dumps(res))
