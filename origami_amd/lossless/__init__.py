from origami_amd.lossless.chunking import PlannedChunk, plan_head_channel_chunks
from origami_amd.lossless.cpu_qat import CpuLosslessCodec

__all__ = ["CpuLosslessCodec", "PlannedChunk", "plan_head_channel_chunks"]
