"""Entry file `kernel.py::run` for the gdn_decode_qk4_v8_d128_k_last definition.

Loaded by path (FlashInfer-Bench style); forwards to the package's decode
operator, which runs the gfx950 HIP kernels of libgdn_hip.so.
"""

import importlib.util
import sys
from pathlib import Path


def _package():
    name = "track_c_gdn_amd"
    if name not in sys.modules:
        root = Path(__file__).resolve().parent.parent
        spec = importlib.util.spec_from_file_location(
            name, root / "__init__.py", submodule_search_locations=[str(root)])
        mod = importlib.util.module_from_spec(spec)
        sys.modules[name] = mod
        spec.loader.exec_module(mod)
    return importlib.import_module(name + ".decode")


_op = _package()
run = _op.run
run_dps = _op.run_dps
