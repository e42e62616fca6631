"""bigsmall_amd — MI355X-native decode engine for BigSmall .bs containers.

Drop-in for the reference's decode path (bigsmall.decoder, codec_registry,
container readers, StreamingLoader / BigSmallStreamingModel, CompressedKVCache):
the same entry points, with every decode running as HIP kernels on the GPU.
"""
__version__ = "3.12.0+mi355x"
