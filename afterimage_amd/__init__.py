"""afterimage_amd: MI355X-native lossless BF16 weight decoder for Afterimage's
compressed-store format. See afterimage_amd.runtime for the decode API."""
__version__ = "0.1.0"
