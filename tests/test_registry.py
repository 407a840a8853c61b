"""The registration a maintainer adds to the reference's ``vsa`` package.

The reference exposes each GPU backend as a lazy loader in ``vsa/__init__.py``
(vsa/__init__.py:28-69: a plain function that imports the backend module on
the first call).  This test writes a small stand-in ``vsa`` package of that
shape into a temporary directory, with the two loaders of the MI355X backend
exactly as the integration notes give them, imports it next to
``vsa_mi355x`` (the names must not collide), and checks that the loaders
resolve and raise the reference's ``ValueError`` texts (common.py:97-134) on
CPU tensors.  No GPU is needed: validation runs before any kernel.
"""

import importlib
import os
import subprocess
import sys
import textwrap

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# The loaders as a maintainer would append them to the reference's vsa/__init__.py.
LOADERS = textwrap.dedent('''
    def mi355x_vsa(*args, **kwargs):
        from vsa_mi355x.mi355x import mi355x_vsa as _impl
        return _impl(*args, **kwargs)


    def mi355x_sparse_attention(*args, **kwargs):
        from vsa_mi355x.mi355x import mi355x_sparse_attention as _impl
        return _impl(*args, **kwargs)
''')


def _stub_package(tmp_path):
    pkg = tmp_path / "vsa"
    pkg.mkdir()
    # A stand-in for the reference's package: eager pure-torch names plus lazy
    # backend loaders (only the loader shape matters here).
    (pkg / "__init__.py").write_text(
        '"""Stand-in for the reference vsa package (lazy backend loaders)."""\n'
        "__all__ = ['mi355x_vsa', 'mi355x_sparse_attention']\n" + LOADERS)
    return tmp_path


@pytest.fixture
def registry(tmp_path, monkeypatch):
    monkeypatch.syspath_prepend(str(_stub_package(tmp_path)))
    monkeypatch.syspath_prepend(os.path.join(ROOT, "simple-vsa_amd"))
    for name in [m for m in sys.modules if m == "vsa" or m.startswith("vsa.")]:
        monkeypatch.delitem(sys.modules, name)
    return importlib.import_module("vsa")


def test_stub_registry_resolves_without_loading_the_backend(registry):
    assert callable(registry.mi355x_vsa) and callable(registry.mi355x_sparse_attention)
    assert registry.__file__.endswith(os.path.join("vsa", "__init__.py"))
    import vsa_mi355x
    assert vsa_mi355x.__name__ != registry.__name__


@pytest.mark.parametrize("case, pattern", [
    ("divisible", "divisible"),
    ("vbs_length", "variable_block_sizes"),
    ("q_vbs_length", "q_variable_block_sizes"),
    ("topk", "topk"),
    ("cpu", "GPU tensors"),
])
def test_registry_mi355x_vsa_raises_reference_texts(registry, case, pattern):
    # tests/test_torch_vsa.py:112-130 of the reference match "divisible",
    # "variable_block_sizes" and "topk".
    be = 4
    s = 10 if case == "divisible" else 12
    q = torch.randn(1, 1, s, 8)
    vbs = torch.full((3,), be)
    qvbs = torch.full((2 if case == "q_vbs_length" else 3,), be)
    if case == "vbs_length":
        vbs = torch.full((2,), be)
    topk = 4 if case == "topk" else 1
    with pytest.raises(ValueError, match=pattern):
        registry.mi355x_vsa(q, q, q, vbs, qvbs, topk, (1, 1, be))


def test_registry_sparse_attention_raises_on_cpu_tensors(registry):
    q = torch.randn(1, 1, 8, 8)
    sel = torch.zeros(1, 1, 2, 1, dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU tensors"):
        registry.mi355x_sparse_attention(q, q, q, sel, torch.full((2,), 4), block_size=(1, 1, 4))


def test_integration_snippet_matches_the_tested_loaders():
    # The loader block in INTEGRATION.md is the one this test registers.
    with open(os.path.join(ROOT, "INTEGRATION.md")) as f:
        text = f.read()
    for line in LOADERS.strip().splitlines():
        if line.strip():
            assert line in text, line


def test_registry_in_a_fresh_interpreter(tmp_path):
    # As a user would run it: only PYTHONPATH, no test scaffolding.
    root = _stub_package(tmp_path)
    env = dict(os.environ, PYTHONPATH=os.pathsep.join(
        [str(root), os.path.join(ROOT, "simple-vsa_amd")]))
    code = ("import torch, vsa\n"
            "q = torch.randn(1, 1, 12, 8)\n"
            "try:\n"
            "    vsa.mi355x_vsa(q, q, q, torch.full((2,), 4), torch.full((3,), 4), 1, (1, 1, 4))\n"
            "except ValueError as e:\n"
            "    print('ValueError:', e)\n")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=300, cwd=str(tmp_path))
    assert out.returncode == 0, out.stderr
    assert "ValueError: variable_block_sizes must have length 3, got 2" in out.stdout
