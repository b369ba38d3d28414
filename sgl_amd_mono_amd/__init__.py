"""An MI355X-native decoder-layer monokernel for SGLang's ``amd`` monokernel backend.

Hand-written gfx950 HIP launches (``csrc/``, built into ``libmono_gfx950.so`` behind the
C-ABI of ``include/mono.h``) run one GPU's share of a DeepSeek-V3.2-shaped decoder layer
with an FP4 indexer; ``spec`` holds the SGLang spec and its forward. SGLang loads the
package as a general plugin through the ``sglang.srt.plugins`` entry point in
``pyproject.toml``, which runs ``register_specs`` (the reference's plugin surface,
sgl_amd_mono/__init__.py:1-55, pyproject.toml:15-17).
"""

__version__ = "0.1.0"

# the monokernel backend every spec registers under (sgl_amd_mono/__init__.py:15)
BACKEND = "amd"
# each spec by (HF architecture, model type); its module imports only when a server
# runs this backend
SPECS = {
    ("DeepseekV32ForCausalLM", "deepseek_v32"): "sgl_amd_mono_amd.spec:SPEC",
}


def _registry():
    """SGLang's spec registry module (the plugin-kernels path, or the older
    ``srt.monokernels`` one)."""
    try:
        from sglang.kernels.plugin_kernels.amd import spec
    except ModuleNotFoundError:
        from sglang.srt.monokernels import spec
    return spec


def register_specs() -> None:
    """The plugin entry point, which SGLang runs in every process."""
    reg = _registry()
    for (architecture, model_type), path in SPECS.items():
        reg.register(backend=BACKEND, architecture=architecture, path=path, model_type=model_type)
