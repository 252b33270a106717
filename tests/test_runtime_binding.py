"""The package swap the unchanged reference runtime binds through (no GPU needed).

``minimaxh3_amd.install_as_kernels()`` aliases this package's kernels as the top-level
``kernels`` package.  The runtime's own import statements must then resolve to this
implementation; they are executed here verbatim (the lines of runtime/model_manager.py:14-16,
runtime/lora.py:18, runtime/generator.py:10-11 and runtime/step_cache.py:6).
"""
import sys

import pytest

import minimaxh3_amd
from minimaxh3_amd.kernels import attention_router, fp8_attention, fp8_linear

# (reference file:line, the statement as it stands there)
RUNTIME_IMPORTS = [
    ("runtime/model_manager.py:14", "from kernels import attention_router"),
    ("runtime/model_manager.py:15", "from kernels.attention_router import denoiser_scope, instrument_transformer"),
    ("runtime/model_manager.py:16", "from kernels.fp8_linear import convert_transformer_to_fp8, find_primary_block_list"),
    ("runtime/lora.py:18", "from kernels.fp8_linear import FP8Linear, apply_lora_adapters"),
    ("runtime/generator.py:10", "from kernels import attention_router"),
    ("runtime/generator.py:11", "from kernels.attention_router import denoiser_scope"),
    ("runtime/step_cache.py:6", "from kernels.fp8_linear import find_primary_block_list"),
]


@pytest.fixture
def installed():
    saved = {k: v for k, v in sys.modules.items() if k == "kernels" or k.startswith("kernels.")}
    for k in saved:
        del sys.modules[k]
    minimaxh3_amd.install_as_kernels()
    try:
        yield
    finally:
        for k in [k for k in sys.modules if k == "kernels" or k.startswith("kernels.")]:
            del sys.modules[k]
        sys.modules.update(saved)


@pytest.mark.parametrize("where,stmt", RUNTIME_IMPORTS, ids=[w for w, _ in RUNTIME_IMPORTS])
def test_runtime_import_statements_resolve_to_this_package(installed, where, stmt):
    ns: dict = {}
    exec(stmt, ns)  # the runtime's statement, unchanged
    names = [n.strip() for n in stmt.split(" import ")[1].split(",")]
    assert names and all(n in ns for n in names), (where, names)
    for n in names:
        obj = ns[n]
        mod = getattr(obj, "__module__", None) or getattr(obj, "__name__", "")
        assert mod.startswith("minimaxh3_amd.kernels"), (where, n, mod)


def test_runtime_modules_share_state_with_the_package(installed):
    """The runtime configures the router it imported (generator.py:180-184); the same module
    object serves the package's own calls, and FP8Linear is the class the LoRA registry checks
    with isinstance (runtime/lora.py:209)."""
    ns: dict = {}
    exec("from kernels import attention_router", ns)
    exec("from kernels.fp8_linear import FP8Linear", ns)
    import kernels.fp8_attention as kfa
    assert ns["attention_router"] is attention_router
    assert ns["FP8Linear"] is fp8_linear.FP8Linear and kfa is fp8_attention
    saved = (attention_router.enabled, attention_router.repair_tau, attention_router.min_seq)
    try:
        ns["attention_router"].configure(enabled=True, repair_tau=0.5, min_seq=1234)
        assert (attention_router.enabled, attention_router.repair_tau, attention_router.min_seq) == (True, 0.5, 1234)
    finally:
        attention_router.configure(*saved)
