"""Host-side sanitizer run of the C ABI (helper of tests/test_capi_asan.py, not a test module).

Loads the host AddressSanitizer + UndefinedBehaviorSanitizer build of libzmoe_hip
(``build_lib.py --asan``) through the package's own ctypes binding, without torch, and
calls every entry point that include/zmoe.h declares with null device pointers and
size arguments from {0, 1, -1, 2^31 - 1, 2^40, 2^62} (all equal, and each pair of size
arguments extreme with the others 1), element-type arguments 0 (f32) and 1 (bf16).
Every call must return a status code, and the pure host functions (workspace sizes,
status strings) must give consistent answers. The host code then has to reject
every such call with a status before touching memory: no out-of-bounds access, no
signed overflow in size arithmetic (the sanitizer runtime, preloaded by the caller,
aborts the process on either). No device memory is touched and nothing is launched
that could run: every device pointer is null, and there is no GPU where the CPU tests
run.

    LD_PRELOAD=<libclang_rt.asan-x86_64.so> python tests/asan_host_driver.py <library> <zmoe/_lib.py> <zmoe.h>
"""

from __future__ import annotations

import ctypes
import importlib.util
import itertools
import re
import sys


def load_binding(lib_path: str, binding_path: str):
    spec = importlib.util.spec_from_file_location("zmoe_lib_standalone", binding_path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    mod.LIB_PATH = lib_path
    return mod, mod.load()


def parameter_names(header: str) -> dict[str, list[str]]:
    """Parameter names of every zmoe_* prototype in the header."""
    text = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(zmoe_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        params = [p.strip() for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = [re.findall(r"[A-Za-z_][A-Za-z0-9_]*", p)[-1] for p in params]
    return out


SIZES = [0, 1, -1, 0x7FFFFFFF, 1 << 40, 1 << 62]
HOST_ONLY = {"zmoe_abi_version", "zmoe_status_string", "zmoe_last_error", "zmoe_sort_error_flag"}


def main() -> int:
    lib_path, binding_path, header = sys.argv[1:4]
    L, lib = load_binding(lib_path, binding_path)
    names = parameter_names(header)
    assert sorted(names) == sorted(L.SIGNATURES), "header and binding disagree"

    # pure host functions
    assert lib.zmoe_abi_version() == 3
    for s in range(-2, 9):
        assert isinstance(lib.zmoe_status_string(s), bytes)
    for R, E in itertools.product([-(1 << 62), -1, 0, 1, 1 << 31, 1 << 62, (1 << 63) - 1], [-1, 0, 1, 1024, 1 << 30]):
        lib.zmoe_sort_workspace_bytes(R, E)
    for N, K, S in itertools.product([-1, 0, 1, 1 << 29, 1 << 40, 1 << 62], [-1, 0, 1, 1 << 40, 1 << 62],
                                     [-1, 0, 1, 64, 1 << 30]):
        lib.zmoe_dense_wgrad_workspace_bytes(N, K, S)
    for E, m, n in itertools.product([-1, 0, 1, 1 << 40, (1 << 63) - 1], [-1, 1, 1 << 20, 1 << 40, 1 << 62],
                                     [-1, 1, 1 << 20, 1 << 40, 1 << 62]):
        lib.zmoe_newton_schulz5_workspace_bytes(E, m, n)

    I64, I32, SZ = ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
    calls = 0
    for name, (res, argtypes) in sorted(L.SIGNATURES.items()):
        if name in HOST_ONLY or name.endswith("_workspace_bytes"):
            continue
        fn = getattr(lib, name)
        pnames = names[name]
        size_pos = [i for i, t in enumerate(argtypes) if t in (I64, I32, SZ) and "dtype" not in pnames[i]]
        dtype_pos = [i for i, t in enumerate(argtypes) if t is I32 and "dtype" in pnames[i]]

        def call(sizes: dict[int, int], dt: int) -> None:
            nonlocal calls
            args = []
            for i, t in enumerate(argtypes):
                if i in dtype_pos:
                    args.append(dt)
                elif i in sizes:
                    v = sizes[i]
                    if t is I32:
                        v = max(min(v, 0x7FFFFFFF), -0x80000000)
                    elif t is SZ:
                        v = v & ((1 << 64) - 1)
                    args.append(v)
                elif t in (ctypes.c_float, ctypes.c_double):
                    args.append(1.0)
                else:
                    args.append(None)  # device pointers and the stream
            rc = fn(*args)
            calls += 1
            assert 0 <= rc <= 6, (name, args, rc)
            if rc:
                assert lib.zmoe_last_error(), name

        for dt in (0, 1):
            for v in SIZES:
                call({i: v for i in size_pos}, dt)
            for i, j in itertools.combinations(size_pos, 2):
                for v in (-1, 1 << 40, 1 << 62):
                    call({**{p: 1 for p in size_pos}, i: v, j: v}, dt)
    print(f"asan host driver: {calls} calls, no report", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
