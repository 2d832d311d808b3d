"""smlm_hip: the product-key-memory lookup of re133/sparse-memory-lm on MI355X (gfx950).

    smlm_hip.kernels  forward kernel API of smlm/kernels.py (pk_select, bag_forward, bag_infer, quantize_q4) plus
                      pk_scores and the int8 table format, backed by libsmlm_pkm.so (include/smlm_pkm.h)
    smlm_hip.pkm      ProductKeyMemory (module API of smlm/pkm.py, impl="hip")
    smlm_hip.model    ModelConfig / Transformer (entry points of smlm/model.py) + whole-step graph decode
    smlm_hip.build    hipcc build of libsmlm_pkm.so
"""
__all__ = ["kernels", "pkm", "model"]
