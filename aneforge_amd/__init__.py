"""aneforge_amd: an MI355X-native (gfx950 HIP) rebuild of ANEForge's quantized-decode hot path,
behind the reference's Python API."""
__version__ = "0.1.0"
