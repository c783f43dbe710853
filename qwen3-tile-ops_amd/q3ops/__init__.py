"""q3ops — MI355X (gfx950) HIP implementation of qwen3-tile-ops' Qwen3 W8A8
forward path, behind the reference's operator surface.

    import sys; sys.path.insert(0, "<repo>/qwen3-tile-ops_amd")
    import q3ops
    lay = q3ops.Layout(q3ops.ModelShape(layers=1, vocab=1024))
    m = q3ops.Model(lay, init=q3ops.InitConfig())
    m.generate()

Submodules: layout (pqwf blob layout + random-init writer), ops (one wrapper
per kernels/*.h operator), model (forward_chunk / greedy generate).  The
operator and model modules need torch with a ROCm device; layout is host-only.
"""
from ._lib import LIB_PATH, LM_ARGMAX, LM_LOGITS, LM_NONE, Q3Error, lib  # noqa: F401
from .layout import (CONFIGS, InitConfig, Layout, ModelShape, init_random_blob,  # noqa: F401
                     quantize_rows_host)


def __getattr__(name):
    # torch is only needed by the device-side modules: import them lazily
    if name == "Model":
        import importlib
        return importlib.import_module(".model", __name__).Model
    raise AttributeError(name)
