"""MI355X-native NSN packed-KV hot path (gfx950 HIP kernels behind a C-ABI)."""
