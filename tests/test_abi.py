"""The C ABI: libhsd.so loads, exports exactly what include/hsd.h declares, and its
host-side argument checks return the documented error codes (no kernel is launched, so
these run without a GPU)."""
import ctypes
import os
import re

import pytest

from hsd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hsd.h")


def header_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(hsd_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = N.lib()
    declared = header_functions()
    assert len(declared) >= 17
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/hsd.h but not exported"
    assert set(declared) == set(N.EXPORTS), "the ctypes signature table must cover the header exactly"
    assert lib.hsd_abi_version() == 1


def header_arities():
    src = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(hsd_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", src):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_ctypes_signatures_match_header_arity():
    ar = header_arities()
    assert set(ar) == set(N.EXPORTS)
    for name, (_, argtypes) in N._SIGS.items():
        assert len(argtypes) == ar[name], f"{name}: ctypes has {len(argtypes)} args, header {ar[name]}"


def test_argument_errors_are_reported():
    lib = N.lib()
    assert lib.hsd_permute_nibbles(None, None, 1, 8, 1, None) == -1
    assert b"null" in lib.hsd_last_error()
    dummy = ctypes.c_void_p(16)
    assert lib.hsd_permute_nibbles(dummy, dummy, 1, 12, 1, None) == -2          # rows % 8
    assert b"multiple of 8" in lib.hsd_last_error()
    args = [dummy, 0, dummy, dummy] + [dummy] * 6 + [dummy, 0]
    # D not a multiple of 128
    assert lib.hsd_sparse_down_decode(*args, 1, 200, 1856, 3712, 6, 128, 0, None, None, dummy, 1 << 30, None) == -2
    # misaligned scales
    odd = ctypes.c_void_p(18)
    args2 = [dummy, 0, dummy, dummy, dummy, odd] + [dummy] * 4 + [dummy, 0]
    assert lib.hsd_sparse_down_decode(*args2, 1, 2688, 1856, 3712, 6, 128, 0, None, None, None, 0, None) == -4
    # front end: misaligned scales (each of the four arrays is loaded 16 bytes at a time)
    for i in range(4):
        sc = [dummy] * 4
        sc[i] = odd
        assert lib.hsd_moe_up_relu2(dummy, 0, dummy, dummy, sc[0], sc[1], dummy, sc[2], sc[3], dummy,
                                    1, 2688, 1856, 3712, 6, 128, None, None, None) == -4
    assert lib.hsd_mamba_verify(*([dummy, 10304] * 3), *([dummy] * 9), 4, dummy, 0,
                                3, 64, 64, 64, 8, 512, 1e-5, 0.0, 1e30, None, dummy, 1 << 20, None) == -2  # N != 128
    assert lib.hsd_mamba_select_row(dummy, None, 4, 3, 4, None, None) == -1       # n_keep > L
    assert lib.hsd_mamba_select_row(dummy, None, 1, 4, 4, None, None) == -2       # L >= nslab
    assert lib.hsd_prefill_gemm(*([dummy] * 14), 0, 512, 2688, 1856, 3712, 6, 128, 48, 240, 3712,
                                dummy, 1 << 30, None) == -2                          # tt = 48
    assert lib.hsd_prefill_gemm(*([dummy] * 14), 0, 512, 2688, 1856, 4096, 6, 128, 32, 240, 4096,
                                dummy, 1 << 30, None) == -2                          # FS > 4032


def test_workspace_sizes():
    lib = N.lib()
    # 32 parts per token row (4 per routed slot of 29 groups, 8 for the shared expert's 58,
    # 8 groups each) x D fp32 partials
    assert lib.hsd_sparse_down_workspace_bytes(1, 2688, 1856, 3712, 6) == 32 * 2688 * 4
    assert lib.hsd_sparse_down_workspace_bytes(3, 2688, 1856, 3712, 6) == 3 * 32 * 2688 * 4
    assert lib.hsd_prefill_num_tiles(512, 6, 128, 32) == 240
    assert lib.hsd_prefill_num_tiles(512, 6, 128, 64) == 184
    assert lib.hsd_prefill_num_tiles(2048, 6, 128, 32) == 576
    # partials [T*7, D] f32, then per tile: group starts (59), padded rows (16 per k-block,
    # 4*58+8 k-blocks), A fragments (1 KiB per k-block), correction fragments (4 x 4 KiB),
    # the GEMM's block schedule (21 column blocks per tile), the staging kernel's dump row
    def al(x):
        return (x + 255) // 256 * 256
    kb = 4 * 58 + 8
    want = (al(512 * 7 * 2688 * 4) + al(240 * 59 * 4) + al(240 * 16 * kb * 4) + al(240 * kb * 1024)
            + al(240 * 4 * 4 * 1024) + al(240 * 21 * 8) + al(256 * 16))
    assert lib.hsd_prefill_gemm_workspace_bytes(512, 2688, 1856, 3712, 6, 128, 32) == want
    assert lib.hsd_prefill_gemm_workspace_bytes(512, 2688, 1856, 3712, 6, 128, 48) == 0
    assert lib.hsd_mamba_workspace_bytes(3, 64, 64) == 3 * 4096 * 4


def test_python_layer_refuses_cpu_tensors():
    import torch
    with pytest.raises(N.HSDError):
        N.ptr(torch.zeros(4))


BUNDLER = "/opt/rocm/llvm/bin/clang-offload-bundler"
READELF = "/opt/rocm/llvm/bin/llvm-readelf"


def device_code_objects(d):
    """The gfx950 code objects of libhsd.so (one per source file), unbundled into dir d."""
    import shutil
    import subprocess
    if not (os.path.exists(BUNDLER) and os.path.exists(READELF) and shutil.which("objcopy") and shutil.which("nm")):
        pytest.skip("ROCm LLVM tools or binutils not installed")
    fb = os.path.join(d, "fb.bin")
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", N.LIB_PATH, fb], check=True)
    blob = open(fb, "rb").read()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    starts = [m.start() for m in re.finditer(re.escape(magic), blob)]
    assert starts, "no offload bundle in libhsd.so"
    out = []
    for i, a in enumerate(starts):              # one bundle per object file
        part, dev = os.path.join(d, f"b{i}.bin"), os.path.join(d, f"dev{i}.o")
        with open(part, "wb") as f:
            f.write(blob[a:starts[i + 1] if i + 1 < len(starts) else len(blob)])
        subprocess.run([BUNDLER, "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={part}",
                        f"--output={dev}", "--unbundle"], check=True)
        out.append(dev)
    return out


def test_every_kernel_handle_has_device_code():
    """Each kernel handle the host side of libhsd.so registers names a kernel of its gfx950
    code object. A launch through a handle without one aborts the process in the HIP
    runtime; a template argument whose type has no name (an unnamed enum) mangles
    differently in the host and device compilations and produced exactly that."""
    import subprocess
    import tempfile
    so = N.LIB_PATH
    with tempfile.TemporaryDirectory() as d:
        devsyms = set()
        for dev in device_code_objects(d):
            devsyms |= {ln.split()[-1] for ln in subprocess.run([READELF, "-s", "-W", dev], check=True,
                                                               capture_output=True, text=True).stdout.splitlines()
                        if ln.strip()}
    host = subprocess.run(["nm", so], check=True, capture_output=True, text=True).stdout.splitlines()
    # kernel handles: local data symbols whose names are kernels of the code object's kind
    handles = {ln.split()[2] for ln in host if len(ln.split()) == 3 and ln.split()[1] in "dD"
               and "_GLOBAL__N_1" in ln.split()[2] and "k_" in ln.split()[2]}
    assert handles, "no kernel handles found in libhsd.so"
    missing = sorted(handles - devsyms)
    assert not missing, f"{len(missing)} kernel handles without device code, e.g. {missing[:3]}"


def test_no_kernel_spills_to_scratch():
    """No kernel of libhsd.so keeps registers in scratch memory: every instance's
    private segment is empty (from the code objects' kernel metadata). A spilled
    instance is a slow path a caller could fall onto with an unusual shape."""
    import subprocess
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        kernels, spilled = 0, []
        for dev in device_code_objects(d):
            notes = subprocess.run([READELF, "--notes", dev], check=True, capture_output=True, text=True).stdout
            for ent in notes.split("- .agpr_count")[1:]:
                name = re.search(r"\.name:\s+(\S+)", ent).group(1)
                priv = int(re.search(r"\.private_segment_fixed_size:\s+(\d+)", ent).group(1))
                spill = int(re.search(r"\.vgpr_spill_count:\s+(\d+)", ent).group(1))
                kernels += 1
                if priv or spill:
                    spilled.append((name, priv, spill))
    assert kernels >= 100
    assert not spilled, f"{len(spilled)} kernels use scratch, e.g. {spilled[:3]}"


def test_linear_row_length_limits():
    """hsd_linear refuses 4-bit rows longer than 4096 inputs and bf16 rows longer than 6144
    (HSD_ERR_SHAPE, before any launch)."""
    lib = N.lib()
    d = ctypes.c_void_p(256)
    def call(w_kind, I):
        return lib.hsd_linear(d, I, 0, None, 0, None, 1e-5, d, d, d, w_kind, d, 64, 0, None, 0, None, 0, None, 0,
                              1, 64, I, None)
    assert call(0, 4160) == -2 and b"at most 4096" in lib.hsd_last_error()
    assert call(1, 6152) == -2 and b"at most 6144" in lib.hsd_last_error()


def test_capture_guard_pauses_the_collector():
    """A stream capture runs with the cycle collector off (after one full pass), and the
    collector's state is restored afterwards, also when the body raises."""
    import gc
    assert gc.isenabled()
    with N.capture_guard():
        assert not gc.isenabled()
    assert gc.isenabled()
    with pytest.raises(RuntimeError):
        with N.capture_guard():
            raise RuntimeError("capture failed")
    assert gc.isenabled()
    gc.disable()
    try:
        with N.capture_guard():
            pass
        assert not gc.isenabled()
    finally:
        gc.enable()
