"""MI355X-native KV-cached Whisper decoder token loop (gfx950 HIP kernels
behind a C ABI, with the reference's Decoder/Net surface in C++ above it)."""
