"""The C ABI of libweft_hip, checked without a GPU: the library loads, exports
every function include/weft_hip.h declares, and its self-describing metadata
agrees with the header (pointer count, const-ness, size_t shape count) and
with the reference's ABI rules (lib/Target/Emission/Emitter.h:465-512)."""
from __future__ import annotations

import re
from pathlib import Path

import pytest

from weft_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "weft_hip.h"


def header_functions() -> dict[str, list[str]]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:const\s+)?[\w]+\s*\*?\s*(\w+)\(([^)]*)\);", text, re.M):
        params = [p.strip() for p in m.group(2).replace("\n", " ").split(",") if p.strip() not in ("", "void")]
        out[m.group(1)] = params
    return out


def test_library_loads_and_reports_version():
    lib = _lib.load()
    assert lib.weft_hip_version().decode().startswith("weft_hip")
    assert lib.weft_hip_get_last_error() == 0


def test_every_header_function_is_exported():
    lib = _lib.load()
    funcs = header_functions()
    assert len(funcs) >= 27
    missing = [name for name in funcs if not hasattr(lib, name)]
    assert not missing


def artifact_phase(name: str) -> bool:
    # <symbol>_W_packed_size / <symbol>_W_pack: the artifact functions of a
    # derived weight layout (lib/Target/Emission/Emitter.h:231-272), not kernels
    return name.endswith("_W_packed_size") or name.endswith("_W_pack")


def test_artifact_covers_every_kernel_in_the_header():
    # weft_hip_*: control API; weft_ggml_*: the GGML MUL_MAT boundary
    funcs = {k for k in header_functions()
             if not k.startswith(("weft_hip_", "weft_ggml_")) and not artifact_phase(k)}
    kernels = {k["symbol"] for k in _lib.artifact()["kernels"]}
    assert funcs == kernels


@pytest.mark.parametrize("kernel", _lib.artifact()["kernels"], ids=lambda k: k["symbol"])
def test_artifact_matches_header_prototype(kernel):
    params = header_functions()[kernel["symbol"]]
    ptrs = [p for p in params if "*" in p]
    sizes = [p for p in params if p.startswith("size_t")]
    assert len(ptrs) + len(sizes) == len(params)
    assert len(ptrs) == len(kernel["arguments"])
    assert [p.split()[-1] for p in sizes] == kernel["shape_parameters"]
    for decl, arg in zip(ptrs, kernel["arguments"]):
        name = decl.replace("*", " ").split()[-1]
        assert name == arg["name"]
        assert decl.startswith("const") == (not arg["writable"])
        assert arg["c_type"].startswith("const ") == (not arg["writable"])
        # restrict only on an argument alone in its non-negative alias set
        members = sum(1 for a in kernel["arguments"] if a["alias_set"] == arg["alias_set"])
        assert arg["c_type"].endswith("*restrict") == (members == 1 and arg["alias_set"] >= 0)
        assert arg["storage_bytes"] > 0 and arg["record_elements"] > 0 and arg["alignment"] > 0


def test_decode_kernels_declare_workspace_and_output_groups():
    # alias_groups={"Xq": "workspace", "Y": "output"} in the Weft sources
    for sym in ("production_mul_mat_q4_k_decode", "production_mul_mat_iq2_xxs_decode",
                "production_mul_mat_mxfp4_decode", "production_mul_mat_iq2_xxs_staged"):
        args = {a["name"]: a for a in _lib.kernel_metadata(sym)["arguments"]}
        assert (args["W"]["alias_set"], args["Xq"]["alias_set"], args["Y"]["alias_set"]) == (0, 1, 2)
    args = {a["name"]: a for a in _lib.kernel_metadata("production_mul_mat_q4_0_decode")["arguments"]}
    assert {a["alias_set"] for a in args.values()} == {0}


def test_artifact_phase_functions_pair_with_their_kernels():
    funcs = header_functions()
    for name, params in funcs.items():
        if name.endswith("_W_packed_size"):
            kernel = name[:-len("_W_packed_size")]
            assert kernel in funcs and kernel + "_W_pack" in funcs
            assert [p.split()[-1] for p in params] == ["M", "K"]
            assert [p.split()[-1] for p in funcs[kernel + "_W_pack"]] == ["*source", "*target", "M", "K"]


def test_packed_size_is_computed_on_the_host():
    import ctypes
    lib = _lib.load()
    fn = lib.q4_k_q8_k_gemv_W_packed_size
    fn.restype = ctypes.c_size_t
    fn.argtypes = [ctypes.c_size_t, ctypes.c_size_t]
    assert fn(14336, 4096) == 14336 * 16 * 144
    assert lib.weft_hip_get_last_error() == 0
    # rows must form whole 16-row cohorts, K whole superblocks
    assert fn(14330, 4096) == 0
    assert lib.weft_hip_get_last_error() != 0
    assert fn(32, 300) == 0
    assert lib.weft_hip_get_last_error() != 0


def test_invalid_call_records_an_error_without_a_device():
    lib = _lib.load()
    # K not a multiple of the record: rejected before any HIP call
    lib.row_dequantize_q4_k(None, None, 100)
    assert lib.weft_hip_get_last_error() != 0
    assert lib.weft_hip_get_last_error() == 0


def test_launch_log_is_off_until_a_thread_turns_it_on():
    """A drop-in caller that never reads the log keeps nothing: the log is
    off by default and turning it off empties it."""
    lib = _lib.load()
    was = lib.weft_hip_set_launch_log(0)
    try:
        assert lib.weft_hip_set_launch_log(0) == 0
        assert lib.weft_hip_launch_log(None, 0) == 0
        assert lib.weft_hip_set_launch_log(1) == 0
        assert lib.weft_hip_set_launch_log(1) == 1
    finally:
        lib.weft_hip_set_launch_log(was)


def test_tile_bindings_accept_the_launch_knobs_only():
    """NC and MR retile the GEMV launches, NC and MC the Q4_K GEMM's tiles;
    other meta names have no gfx950 knob (0, no error); a value above
    INT32_MAX or no name is an error."""
    lib = _lib.load()
    try:
        assert lib.weft_hip_set_tile_binding(b"NC", 64) == 1
        assert lib.weft_hip_set_tile_binding(b"MR", 2) == 1
        assert lib.weft_hip_set_tile_binding(b"MC", 32) == 1
        for name in (b"KC", b"NR", b"nc", b""):
            assert lib.weft_hip_set_tile_binding(name, 8) == 0
        assert lib.weft_hip_get_last_error() == 0
        lib.weft_hip_set_tile_binding(b"NC", 1 << 31)
        assert lib.weft_hip_get_last_error() != 0
        lib.weft_hip_set_tile_binding(None, 1)
        assert lib.weft_hip_get_last_error() != 0
    finally:
        lib.weft_hip_clear_tile_bindings()


# ----------------------------------------------- device variables of the library
READELF = Path("/opt/rocm/llvm/bin/llvm-readelf")
OBJCOPY = Path("/opt/rocm/llvm/bin/llvm-objcopy")


def device_code_objects(so: Path) -> list[bytes]:
    """The gfx950 code objects in the library's .hip_fatbin section (one
    clang offload bundle per translation unit)."""
    import struct
    import subprocess
    import tempfile
    with tempfile.TemporaryDirectory() as tmp:
        fat = Path(tmp) / "fatbin"
        subprocess.run([str(OBJCOPY), f"--dump-section=.hip_fatbin={fat}", str(so), str(Path(tmp) / "x")],
                       check=True, capture_output=True)
        data = fat.read_bytes()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    out = []
    at = data.find(magic)
    while at >= 0:
        (count,) = struct.unpack_from("<Q", data, at + len(magic))
        pos = at + len(magic) + 8
        for _ in range(count):
            off, size, tlen = struct.unpack_from("<QQQ", data, pos)
            triple = data[pos + 24:pos + 24 + tlen].decode()
            pos += 24 + tlen
            if "gfx950" in triple:
                out.append(data[at + off:at + off + size])
        at = data.find(magic, at + 1)
    return out


@pytest.mark.skipif(not (READELF.exists() and OBJCOPY.exists()), reason="needs ROCm's llvm-readelf / llvm-objcopy")
def test_host_registered_device_variables_exist_in_the_code_objects():
    """Every __device__ variable the host side registers must survive in the
    device code object: an internal const object that no kernel reads is
    dropped there while the host still registers it, and the HIP runtime then
    aborts the process at the first launch from that code object.  The
    library's variables are the GGML tables and the no-allocation scratch."""
    import subprocess
    import tempfile
    objects = device_code_objects(_lib.LIB_PATH)
    assert objects
    symbols = []
    with tempfile.TemporaryDirectory() as tmp:
        for i, co in enumerate(objects):
            path = Path(tmp) / f"co{i}.o"
            path.write_bytes(co)
            res = subprocess.run([str(READELF), "--syms", "--wide", str(path)], check=True,
                                 capture_output=True, text=True)
            symbols += [line.split() for line in res.stdout.splitlines() if " OBJECT " in line]
    found = {row[-1]: row for row in symbols}
    for needle in ("g_weft_ggml_tables", "scratch"):
        hits = [name for name in found if needle in name and not name.endswith(".kd")]
        assert hits, f"device variable {needle} missing from the code objects"
        for name in hits:
            assert found[name][4] == "GLOBAL", f"{name} is not a global symbol of the code object"


@pytest.mark.skipif(not (READELF.exists() and OBJCOPY.exists()), reason="needs ROCm's llvm-readelf / llvm-objcopy")
def test_no_kernel_spills_to_scratch():
    """Every kernel keeps its state in registers and LDS: a kernel whose
    accumulators went to scratch memory (a private segment) runs tens of
    times slower.  The code objects' kernel metadata states each kernel's
    private segment; the one tolerated is the grouped (MUL_MAT_ID) Q4_K
    GEMM's 12-byte spill of two VGPRs."""
    import re
    import subprocess
    import tempfile
    objects = device_code_objects(_lib.LIB_PATH)
    assert objects
    sizes = {}
    with tempfile.TemporaryDirectory() as tmp:
        for i, co in enumerate(objects):
            path = Path(tmp) / f"co{i}.o"
            path.write_bytes(co)
            res = subprocess.run([str(READELF), "--notes", "--wide", str(path)], check=True,
                                 capture_output=True, text=True)
            for block in re.split(r"\n\s+- \.", res.stdout):
                name = re.search(r"\.name:\s+(\S+)", block)
                seg = re.search(r"\.private_segment_fixed_size:\s+(\d+)", block)
                if name and seg:
                    sizes[name.group(1)] = int(seg.group(1))
    assert len(sizes) > 50
    spilled = {k: v for k, v in sizes.items() if v > 0}
    allowed = {k: v for k, v in spilled.items() if "q4k_mfma_gemm" in k and "ILb1E" in k and v <= 16}
    assert spilled == allowed, spilled
