"""torch_xdna for MI355X: a torch.compile backend whose int8 hot path runs as HIP kernels on one GPU.

    import torch, torch_xdna
    model = torch.compile(model, backend="xdna", options={"policy": "gpu"})

GEMMs against parameters run W8A8 (per-row int8 activations, per-channel int8 weights, int32
accumulate, fp32 dequantize) and 3x3 stride-1 convolutions run as int8 implicit GEMMs with a fused
shift / round / saturate requantize, both on MFMA. The API is the reference torch-xdna's: the
`xdna` backend, Config / set_config, the xdna:: custom ops, report() and stats. Integer results
are bit-identical to the reference's CPU route. See torch_xdna.Config for every option and
torch_xdna.report() for where the work went.
"""

import json

from . import kernels, ops  # noqa: F401  (registers the xdna:: ops)
from .backend import offload_gemms, xdna_backend
from .config import Config, set_config
from .runtime import stats

__all__ = ["Config", "set_config", "xdna_backend", "offload_gemms", "compile", "stats", "report",
           "gpu_available", "npu_available"]
__version__ = "0.1.0"


def _register():
    from torch._dynamo.backends.registry import _BACKENDS, register_backend

    if "xdna" not in _BACKENDS:
        register_backend(xdna_backend, name="xdna")


_register()


def compile(model, **options):
    """torch.compile(model, backend="xdna", options=options)."""
    import torch

    return torch.compile(model, backend="xdna", options=options or None)


def gpu_available() -> bool:
    return kernels.available()


npu_available = gpu_available   # the reference's name


def report(as_json=False):
    """Where the GEMMs and convs ran (calls, seconds, GMACs per device), GPU launches, fallbacks, autotune."""
    d = stats.as_dict()
    if as_json:
        return json.dumps(d, indent=1)
    lines = [f"GPU available: {d['gpu_available']}" +
             (f" ({d['gpu_unavailable_reason']})" if not d["gpu_available"] else "")]
    for dev in sorted(d["calls"]):
        lines.append(f"  {dev:4s}: {d['calls'][dev]} calls, {d['gmacs'][dev]} GMAC, {d['seconds'][dev]} s")
    lines.append(f"  GPU launches: {d['gpu_launches']}")
    for k, v in d["decisions"].items():
        lines.append(f"  auto {k}: {v[0]} (gpu {v[1]} ms, cpu {v[2]} ms)")
    for shape, err in d["fallbacks"]:
        lines.append(f"  fallback {shape}: {err}")
    return "\n".join(lines)
