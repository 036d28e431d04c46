"""MI355X (gfx950) implementation of Alelyon Compute Kit's vq4/v1 path.

``alelyon_compute_kit.vq`` keeps the reference's import path and API;
``alelyon_compute_kit.ack`` is the device/buffer binding of libackvq.so;
``expert_bank`` and ``harness`` are the durable expert store and the
linear-expert driver that call into the vq4 path.
"""
__all__ = ["ack", "vq", "expert_bank", "harness"]
