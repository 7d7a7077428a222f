"""CPU-side checks of the C ABI: the library loads without a GPU and exports every
function include/pcu_rocm.h declares, and the Python binding covers the same set."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for header in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not header.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", header)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(pcu_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_header_declares_the_boundary():
    names = _declared_functions()
    for required in ("pcu_ctx_open", "pcu_strict_matmul", "pcu_strict_sgd", "pcu_strict_mse",
                     "pcu_checked_binary", "pcu_checked_relu", "pcu_checked_relu_backward",
                     "pcu_program_begin", "pcu_program_end"):
        assert required in names


def test_library_exports_every_declared_symbol(pcu_pkg):
    lib_path = pcu_pkg.library_path()
    assert os.path.exists(lib_path), "build the library first (python __graft_entry__.py)"
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = sorted(_declared_functions() - exported)
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_header_and_loads_without_gpu(pcu_pkg):
    from fusion_pcu_amd import _abi
    assert set(_abi.SIGNATURES) >= _declared_functions() - _graph_only()
    lib = pcu_pkg.lib()
    header = open(os.path.join(ROOT, "include", "pcu_rocm.h")).read()
    version = int(re.search(r"#define PCU_ROCM_ABI_VERSION (\d+)", header).group(1))
    assert lib.pcu_abi_version() == version


def test_node_descriptor_layout_matches_the_header():
    """The ctypes mirror of pcu_node_desc has the C layout (compiled with the host compiler
    from the header itself)."""
    import ctypes
    import tempfile
    from fusion_pcu_amd import _abi
    src = ('#include <stdio.h>\n#include <stddef.h>\n#include "pcu_rocm.h"\n'
           'int main(void){printf("%zu %zu %zu", sizeof(pcu_node_desc), '
           'offsetof(pcu_node_desc, options), sizeof(pcu_numerical_options)); return 0;}\n')
    with tempfile.TemporaryDirectory() as d:
        c, exe = os.path.join(d, "layout.c"), os.path.join(d, "layout")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), c, "-o", exe], check=True)
        size, off, osize = map(int, subprocess.run([exe], capture_output=True, text=True,
                                                   check=True).stdout.split())
    assert ctypes.sizeof(_abi.NodeDesc) == size
    assert _abi.NodeDesc.options.offset == off
    assert ctypes.sizeof(_abi.NumericalOptions) == osize


def _graph_only():
    from fusion_pcu_amd import _abi
    return {n for n in _declared_functions() if n not in _abi.SIGNATURES and n.startswith("pcu_graph")}


def test_opening_a_context_without_gpu_fails_loudly(pcu_pkg):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(pcu_pkg.PcuExecutionError):
        pcu_pkg.Context(0)


def test_product_package_never_reaches_the_oracle():
    """No CPU fallback: no module of the product package imports `oracle`, no native source
    includes or loads anything from it, and importing the package with its graph front end
    leaves `oracle` unimported (checked in a fresh interpreter)."""
    import ast
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    pkg = os.path.join(root, "fusion-pcu_amd")
    for name in os.listdir(pkg):
        if name.endswith(".py"):
            tree = ast.parse(open(os.path.join(pkg, name)).read())
            for node in ast.walk(tree):
                if isinstance(node, ast.Import):
                    assert not any(a.name.split(".")[0] == "oracle" for a in node.names), name
                elif isinstance(node, ast.ImportFrom):
                    assert (node.module or "").split(".")[0] != "oracle", name
    csrc = os.path.join(pkg, "csrc")
    for name in os.listdir(csrc):
        text = open(os.path.join(csrc, name)).read()
        assert "oracle/" not in text and "_ref/" not in text, name
    probe = (
        "import importlib.util, os, sys\n"
        f"pkg = {pkg!r}\n"
        "spec = importlib.util.spec_from_file_location('fusion_pcu_amd', os.path.join(pkg, '__init__.py'), "
        "submodule_search_locations=[pkg])\n"
        "m = importlib.util.module_from_spec(spec); sys.modules['fusion_pcu_amd'] = m; spec.loader.exec_module(m)\n"
        "import fusion_pcu_amd.graph, fusion_pcu_amd.synthetic\n"
        "assert not any(k == 'oracle' or k.startswith('oracle.') for k in sys.modules), 'oracle imported'\n")
    subprocess.run([sys.executable, "-c", probe], check=True, cwd="/", timeout=120)
