"""bigsmall_amd — MI355X-native decode engine for BigSmall .bs containers.

Drop-in for the reference's decode path, with every decode running as HIP
kernels on the GPU:
    compress(src, dst)                      -> .bs in the GPU format (bf16_chunked_v1)
    decompress(src, dst=None)               -> dict[str, np.ndarray]
    load(src, device="cuda")                -> dict[str, torch.Tensor] in HBM
    info(src), verify(src)
    StreamingLoader, BigSmallStreamingModel -> layer-at-a-time decode with prefetch
    streaming_model.StreamingGPT2           -> GPT-2 run block by block from a StreamingLoader
    decompress_layers(src, [i, ...])        -> only the named layers
    decompress_delta(delta, base), load_delta(delta, base) -> a fine-tune from its XOR delta
    CompressedKVCache                       -> KV entries and blocks decoded on the GPU
    codec_registry.register_codec / get_codec / auto_select_codec
    compress_for_hub(model_dir, out_dir), from_pretrained(path) -> multi-shard .bs models + index
    migrate.migrate(path)                   -> re-encode a container into the GPU formats where smaller
"""
__version__ = "3.12.0+mi355x"

from .container import info
from .decoder import decompress, decompress_delta, load, load_delta
from .encoder import compress
from .exceptions import BigSmallVersionError, DecodeError
from .hub import compress_for_hub, from_pretrained
from .kv_cache_manager import CompressedKVCache
from .streaming import StreamingLoader, decompress_layers
from .verify import verify


def __getattr__(name):
    # transformers/accelerate are only needed by the streaming model
    if name == "BigSmallStreamingModel":
        from .streaming_inference import BigSmallStreamingModel
        return BigSmallStreamingModel
    if name == "StreamingGPT2":
        from .streaming_model import StreamingGPT2
        return StreamingGPT2
    raise AttributeError(name)


__all__ = ["compress", "decompress", "load", "info", "verify", "StreamingLoader", "BigSmallStreamingModel",
           "decompress_layers", "decompress_delta", "load_delta",
           "CompressedKVCache", "BigSmallVersionError", "DecodeError", "compress_for_hub", "from_pretrained",
           "__version__"]
