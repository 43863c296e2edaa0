"""GRINQH quantization for vLLM on MI355X (gfx950).

``register()`` is the ``vllm.general_plugins`` entry point (same name and
target as the reference, pyproject.toml:20-21 / grinqh/__init__.py:1-2):
importing ``grinqh.grinqh`` registers the ``"grinqh"`` quantization config and
the ``torch.ops.grinqh.gemm_or_gemv`` op.
"""


def register():
    from . import grinqh  # noqa: F401  (runs @register_quantization_config)
