"""MI355X-native Qwen3.5-4B int4 decode path: gfx950 HIP kernels behind deltaforge's slot surface."""

__version__ = "0.1.0"
