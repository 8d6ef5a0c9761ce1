"""Engine plugins: aklr_amd as an aiter kernel-plugin provider, enabled from sglang's or vLLM's
plugin entry points (aklr/plugins/README.md:1-57 of the reference)."""
