"""KV-cache movement operators of the ROCm HIP backend."""
