"""Load reference modules for golden-vector generation (this container only).

The reference tree is not importable as-is here: its package ``__init__`` files pull
in e3nn-based modes, and ``e3nn`` (pinned ``>=0.4.4,<0.6.0``, ``setup.py:81``) and
``torch_scatter`` (``>=2.0.9``, ``setup.py:93``) are absent from the image.  This
loader

* registers bare package objects for ``molecular_force_field``, ``.models`` and
  ``.utils`` whose ``__path__`` points into the reference tree, so individual
  module files load without executing the package ``__init__`` files;
* provides ``e3nn.math.soft_one_hot_linspace`` from the oracle's restatement of
  e3nn's published formula (so golden vectors do not pin that function: it stays
  "parity unpinned", see ``oracle/radial.py``);
* provides ``torch_scatter.scatter`` as the reference's own index_add fallback
  (``utils/scatter.py:63-116``).

No compiled reference artefact is loaded: ``molecular_force_field._C_ictd_tp`` is
pre-registered as an empty module without the extension's functions, which the
reference treats as "extension unavailable" (``models/ictd_irreps_cuda.py:9-40``).
"""

from __future__ import annotations

import importlib
import os
import sys
import types

REF_ROOT = os.environ.get("FSCTEP_REFERENCE_ROOT", "/root/reference")


def setup() -> None:
    if "molecular_force_field" in sys.modules and getattr(sys.modules["molecular_force_field"], "_golden_stub", False):
        return
    here = os.path.dirname(os.path.abspath(__file__))
    repo = os.path.dirname(os.path.dirname(here))
    if repo not in sys.path:
        sys.path.insert(0, repo)
    from oracle.radial import soft_one_hot_linspace

    pkg_root = os.path.join(REF_ROOT, "molecular_force_field")
    for name, sub in (("molecular_force_field", ""), ("molecular_force_field.models", "models"),
                      ("molecular_force_field.utils", "utils")):
        m = types.ModuleType(name)
        m.__path__ = [os.path.join(pkg_root, sub) if sub else pkg_root]
        m._golden_stub = True
        sys.modules[name] = m
    ext = types.ModuleType("molecular_force_field._C_ictd_tp")
    sys.modules["molecular_force_field._C_ictd_tp"] = ext
    sys.modules["molecular_force_field"]._C_ictd_tp = ext

    e3nn = types.ModuleType("e3nn")
    e3nn_math = types.ModuleType("e3nn.math")
    e3nn_math.soft_one_hot_linspace = (
        lambda x, start, end, number, basis=None, cutoff=None:
        soft_one_hot_linspace(x, start, end, number, basis=basis, cutoff=bool(cutoff)))
    e3nn.math = e3nn_math
    sys.modules["e3nn"] = e3nn
    sys.modules["e3nn.math"] = e3nn_math

    scat = importlib.import_module("molecular_force_field.utils.scatter")
    ts = types.ModuleType("torch_scatter")
    ts.scatter = scat.scatter
    sys.modules["torch_scatter"] = ts
    import warnings
    warnings.filterwarnings("ignore", message="torch_scatter is not available")


def load(module: str):
    setup()
    return importlib.import_module(module)
