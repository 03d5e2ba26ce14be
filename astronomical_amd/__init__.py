"""MI355X-native sorted mixture-of-experts block (HIP kernels behind a C ABI)."""
