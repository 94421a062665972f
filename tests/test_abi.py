"""The C ABI library and the extension module: load, exports, argument errors (CPU)."""
import ctypes
import os
import re

import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "batmobile-evo_amd", "lib", "libbatmobile_hip.so")
HEADER = os.path.join(REPO, "include", "batmobile_hip.h")


def _declared_functions():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    names = re.findall(r"^\s*(?:int|void|size_t)\s+(\w+)\s*\(", txt, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_path():
    names = _declared_functions()
    for n in ("batteries_spherical_harmonics", "batteries_tensor_product_l3",
              "batteries_tensor_product_backward_l3", "batteries_sh_tp_scatter_csr",
              "batteries_fused_sh_tp_simple", "batteries_edge_index_to_csr",
              "neighbor_list_cuda", "neighbor_list_free", "neighbor_list_estimate_memory"):
        assert n in names


def test_library_loads_and_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB)
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_reference_named_neighbor_library():
    """libbatteries_neighbor.so, the name the reference's ctypes callers load
    (benchmarks/benchmark_neighbor_list.py:18-22, benchmark_e2e_mace.py:38), exports the
    reference's three neighbor-list symbols."""
    nl = ctypes.CDLL(os.path.join(REPO, "batmobile-evo_amd", "lib", "libbatteries_neighbor.so"))
    for n in ("neighbor_list_cuda", "neighbor_list_free", "neighbor_list_estimate_memory"):
        assert hasattr(nl, n)
    nl.neighbor_list_estimate_memory.restype = ctypes.c_size_t
    nl.neighbor_list_estimate_memory.argtypes = [ctypes.c_int64, ctypes.c_float, ctypes.c_float]
    assert nl.neighbor_list_estimate_memory(1000, 0.05, 5.0) > 0


def test_noalloc_backward_rejects_oversize_before_any_device_call():
    """The no-allocation backward refuses a call whose grad_W partials exceed its static
    scratch (24 MiB) with BATMOBILE_HIP_ERR_SCRATCH, before touching the device."""
    lib = ctypes.CDLL(LIB)
    f = lib.batteries_tensor_product_backward_l3_noalloc
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 7 + [ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_void_p]
    one = ctypes.c_void_p(16)  # never dereferenced: the size check comes first
    assert f(one, one, one, one, None, None, one, 100000, 1024, 1024, None) == -4


def test_noalloc_scratch_holds_every_claimed_shape():
    """The header's claim: the no-allocation backward's grad_W partials fit its 24 MiB
    scratch for every N whenever 3 * ceil(C_in/16) * ceil(C_out/64) <= 512.  Swept over N
    from 1 to 10^7 and channel pairs across and at the corners of that region, with the
    host-only workspace-size function (no GPU)."""
    lib = ctypes.CDLL(LIB)
    f = lib.batteries_tensor_product_backward_workspace_bytes
    f.restype = ctypes.c_size_t
    f.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.c_int]
    scratch = 24 << 20
    ns = sorted(set([1, 2, 15, 16, 17, 100, 255, 256, 257, 1000, 4095, 4096, 4097, 20000,
                     65535, 65536, 100003, 10 ** 6, 1234567, 10 ** 7]
                    + [int(round(10 ** (k / 4))) for k in range(29)]))
    pairs = [(256, 256), (16, 10880), (208, 832), (10880, 16), (2720, 64), (16, 64), (1, 1),
             (32, 64), (64, 64), (128, 128), (170, 640), (255, 255), (512, 128), (96, 1088)]
    pairs += [(ci, co) for ci in (1, 7, 16, 31, 48, 100, 160) for co in (1, 33, 64, 65, 500, 1000)]
    checked = 0
    for ci, co in pairs:
        combos = 3 * -(-ci // 16) * -(-co // 64)
        if combos > 512:
            continue
        for n in ns:
            assert f(n, ci, co) <= scratch, (n, ci, co, f(n, ci, co))
            checked += 1
    assert checked > 500
    # just outside the region the partials can exceed it
    assert f(10 ** 6, 1024, 1024) > scratch


def test_host_only_entry_points():
    lib = ctypes.CDLL(LIB)
    assert lib.batteries_get_num_paths_l3() == 34
    info = (ctypes.c_int * 102)()
    lib.batteries_get_path_info_l3(info)
    assert list(info[:9]) == [0, 0, 0, 0, 1, 1, 0, 2, 2]
    lib.neighbor_list_estimate_memory.restype = ctypes.c_size_t
    lib.neighbor_list_estimate_memory.argtypes = [ctypes.c_int64, ctypes.c_float, ctypes.c_float]
    assert lib.neighbor_list_estimate_memory(1000, 0.05, 5.0) > 0
    lib.batteries_neighbor_list_workspace_bytes.restype = ctypes.c_size_t
    lib.batteries_neighbor_list_workspace_bytes.argtypes = [ctypes.c_int64, ctypes.c_void_p,
                                                            ctypes.c_float]
    box = (ctypes.c_float * 3)(20.0, 20.0, 20.0)
    assert lib.batteries_neighbor_list_workspace_bytes(100, box, 5.0) > 0
    bad = (ctypes.c_float * 3)(20.0, -1.0, 20.0)
    assert lib.batteries_neighbor_list_workspace_bytes(100, bad, 5.0) == 0


def test_extension_module_names(bm):
    import _batteries
    import batmobile
    ref_names = ["spherical_harmonics", "spherical_harmonics_inplace", "tensor_product_simple",
                 "tensor_product", "get_tp_path_info", "get_tp_num_paths",
                 "spherical_harmonics_backward", "tensor_product_simple_backward",
                 "tensor_product_backward", "edge_index_to_csr", "fused_message_passing_simple",
                 "fused_message_passing", "fused_sh_tp_simple"]
    for n in ref_names:
        assert getattr(bm, n) is getattr(_batteries, n)
        assert hasattr(batmobile, n)
    for n in ("SphericalHarmonicsFunction", "TensorProductSimpleFunction", "TensorProductFunction",
              "spherical_harmonics_autograd", "tensor_product_autograd"):
        assert hasattr(batmobile, n)
    info = bm.get_tp_path_info()
    assert info.dtype == torch.int32 and tuple(info.shape) == (34, 3) and info.device.type == "cpu"
    assert bm.get_tp_num_paths() == 34


@pytest.mark.parametrize("call", [
    lambda b: b.spherical_harmonics(torch.zeros(4, 3), 3),                       # CPU tensor
    lambda b: b.spherical_harmonics(torch.zeros(4, 3), 7),                       # L range
    lambda b: b.spherical_harmonics(torch.zeros(4, 2), 3),                       # shape
    lambda b: b.spherical_harmonics(torch.zeros(4, 3, dtype=torch.float64), 3),  # dtype
    lambda b: b.tensor_product_simple(torch.zeros(4, 16), torch.zeros(5, 16)),
    lambda b: b.tensor_product(torch.zeros(4, 2, 16), torch.zeros(4, 16), torch.zeros(33, 2, 3)),
    lambda b: b.tensor_product(torch.zeros(4, 2, 16), torch.zeros(4, 16), torch.zeros(34, 3, 3)),
    lambda b: b.tensor_product_backward(torch.zeros(4, 2, 16), torch.zeros(4, 16),
                                        torch.zeros(34, 2, 3), torch.zeros(4, 5, 16)),
    lambda b: b.spherical_harmonics_backward(torch.zeros(4, 3), torch.zeros(4, 15)),
    lambda b: b.fused_sh_tp_simple(torch.zeros(4, 3), torch.zeros(2, 3, 16),
                                   torch.zeros(4, dtype=torch.int32)),
    lambda b: b.edge_index_to_csr(torch.zeros(3, 4, dtype=torch.int64), 5),
    lambda b: b.fused_message_passing(torch.zeros(2, 3, 16), torch.zeros(4, 3), torch.zeros(4, 5),
                                      torch.zeros(3, dtype=torch.int64),
                                      torch.zeros(4, dtype=torch.int64)),
    lambda b: b.sh_tp_scatter_weighted(torch.zeros(4, 3), torch.zeros(2, 3, 16),
                                       torch.zeros(33, 3, 3), torch.zeros(4, dtype=torch.int64),
                                       torch.zeros(3, dtype=torch.int64)),
])
def test_argument_errors_raise_runtime_error(bm, call):
    with pytest.raises(RuntimeError):
        call(bm)


def test_package_fails_loudly_without_the_extension(tmp_path):
    """No CPU fallback: the package copied without its compiled extension refuses to import."""
    import shutil
    import subprocess
    import sys
    pkg = os.path.join(REPO, "batmobile-evo_amd", "python", "batmobile")
    shutil.copytree(pkg, tmp_path / "batmobile", ignore=shutil.ignore_patterns("__pycache__"))
    code = f"import sys; sys.path.insert(0, {str(tmp_path)!r}); import batmobile"
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode != 0
    assert "ImportError" in r.stderr and "not built" in r.stderr


def test_extension_refuses_host_tensors():
    """Host (CPU) tensors are refused with an error, never computed on the CPU."""
    import sys
    import torch
    sys.path.insert(0, os.path.join(REPO, "batmobile-evo_amd", "python"))
    import _batmobile
    with pytest.raises(RuntimeError):
        _batmobile.spherical_harmonics(torch.zeros(4, 3), 3)
    with pytest.raises(RuntimeError):
        _batmobile.tensor_product_simple(torch.zeros(4, 16), torch.zeros(4, 16))
