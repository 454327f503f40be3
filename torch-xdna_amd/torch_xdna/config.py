"""Options of the xdna backend: torch.compile(..., backend="xdna", options={...}) or torch_xdna.set_config.

Every field of the reference's Config (torch_xdna/config.py:11-53 in the reference) is kept with its
name, default and validation, so existing `options=` dicts run unchanged. The device is an MI355X
GPU instead of the XDNA NPU: policy "gpu" forces it, and the reference's "npu" is accepted as an
alias of "gpu".

Fields whose meaning was specific to the NPU are accepted and keep their validation:
  row_buckets    the GPU kernels take any row count without padding; buckets only name the row
                 group in autotune keys (as in the reference's `_choose`).
  tuned_tilings  per-shape tile choices from the shipped MI355X sweep table (torch_xdna/tuned/), or
                 TORCH_XDNA_TUNED; off: the library's built-in tile rule.
  stacks         a Qwen3-0.6B-width transformer stack + linear head on GPU tensors becomes the one op
                 xdna::qwen3_stack (HIP kernels), dispatched per call by the attention mask.
"""

from dataclasses import dataclass, fields, replace

POLICIES = ("auto", "gpu", "npu", "cpu")
FALLBACKS = ("inductor", "eager")
CPU_KERNELS = ("int8", "fp")
PRECISIONS = ("int8", "bf16")


@dataclass(frozen=True)
class Config:
    # Where an offloadable GEMM / conv runs:
    #   auto  GPU for tensors already on the GPU; for host tensors, measure GPU (with the copies)
    #         against the CPU once per (row bucket, N, K) and keep the faster
    #   gpu   always the GPU (CPU only when it is unavailable or a launch fails); "npu" = "gpu"
    #   cpu   never the GPU
    policy: str = "auto"
    # What compiles the rest of the graph: inductor / eager.
    fallback: str = "inductor"
    # Offloaded GEMM math: int8 (W8A8, per-channel weights, per-row activations, int32 accumulate;
    # GPU == CPU bit for bit) or bf16 (the reference's fp32 CPU route).
    precision: str = "int8"
    # A GEMM the GPU does not take runs on the CPU as int8 (the same W8A8 math) or fp (the original
    # linear).
    cpu_kernel: str = "int8"
    # Host-resident GEMMs with fewer rows / MACs stay on the CPU without asking (a launch costs the
    # PCIe copies). Tensors already on the GPU always use the GPU route.
    min_rows: int = 16
    row_buckets: tuple = (128, 256, 512, 1024)
    min_macs: int = 2_000_000
    # Linears that read the same input (q/k/v, gate/up) run as one GEMM.
    fuse: bool = True
    stacks: bool = True
    tuned_tilings: bool = True
    # Check GPU results against the CPU: "first" launch of every GPU program, "always", or "off".
    verify: str = "first"
    verbose: bool = False

    def __post_init__(self):
        assert self.policy in POLICIES, f"policy must be one of {POLICIES}"
        assert self.fallback in FALLBACKS, f"fallback must be one of {FALLBACKS}"
        assert self.cpu_kernel in CPU_KERNELS, f"cpu_kernel must be one of {CPU_KERNELS}"
        assert self.precision in PRECISIONS, f"precision must be one of {PRECISIONS}"
        assert self.verify in ("first", "always", "off"), "verify must be first / always / off"
        assert all(b % 128 == 0 for b in self.row_buckets), "row buckets must be multiples of 128"
        if self.policy == "npu":
            object.__setattr__(self, "policy", "gpu")

    def merged(self, options=None):
        if not options:
            return self
        known = {f.name for f in fields(self)}
        bad = set(options) - known
        assert not bad, f"unknown xdna options {sorted(bad)}; known: {sorted(known)}"
        if "row_buckets" in options:
            options = dict(options, row_buckets=tuple(sorted(options["row_buckets"])))
        return replace(self, **options)


config = Config()


def set_config(**options):
    """Process-wide defaults; per-compile options override them."""
    global config
    config = config.merged(options)
    return config
