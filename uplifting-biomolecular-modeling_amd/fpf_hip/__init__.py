"""fpf_hip -- the FlashPairformer pair-stack hot path on MI355X (gfx950): host-side faces over libfpf_hip.so.

Faces (the reference's provider interfaces, same names and argument meaning):
    fpf_hip.kernels.ln          layer_norm
    fpf_hip.kernels.transition  pack, Weights, transition
    fpf_hip.kernels.trimul      triangle_multiplication, select, WEIGHT_KEYS
    fpf_hip.kernels.triattn     triangle_attention, select
    fpf_hip.attn.pair_fused     pack_triattn_weights, tri_attn_block, pack_transition_weights, transition
    fpf_hip.pairformer          pair_block / pair_stack (the five in-place pair sites per layer)
Every face calls the HIP library and raises when it is missing; nothing here computes on the CPU.
"""
__all__ = ["kernels", "attn", "pairformer"]
