"""MI355X kernels for the Qwen3.6 MoE decode layer and Gated DeltaNet step."""
