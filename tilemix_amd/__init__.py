"""tilemix_amd -- TileMix fused FP16/INT8 prefill attention for MI355X (gfx950).

Mirrors the reference package layout so a caller swaps an import prefix:
``attention.precision_maps`` -> ``tilemix_amd.attention.precision_maps``,
``attention.tilemix_varlen`` -> ``tilemix_amd.attention.tilemix_varlen``,
``attention.triton.tilemix`` -> ``tilemix_amd.attention.hip.tilemix``,
``models.tilemix_llama`` / ``models.tilemix_qwen`` -> ``tilemix_amd.models.*``.
"""

__all__ = ["inject_tilemix_into_llama", "inject_tilemix_into_qwen"]


def __getattr__(name):
    # Model integrations import transformers; load them on first use only.
    if name == "inject_tilemix_into_llama":
        from .models.tilemix_llama import inject_tilemix_into_llama
        return inject_tilemix_into_llama
    if name == "inject_tilemix_into_qwen":
        from .models.tilemix_qwen import inject_tilemix_into_qwen
        return inject_tilemix_into_qwen
    raise AttributeError(name)
