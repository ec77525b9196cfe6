"""MI355X (gfx950) backend for fluidaudio-web's Parakeet FastConformer encoder.

    from fluidaudio_web_amd import createContext, FusedEncoder
    ctx = createContext("hip")
    enc = FusedEncoder(ctx, manifest, fmt="f16")
    frames = enc.encode([mel0, mel1])          # list of [Tsub_i, 1024]

The package directory is `fluidaudio-web_amd/`; import it with
`fluidaudio_web_amd.load()` semantics via the repo's loader (see
__graft_entry__.load_package) or put its parent on sys.path under an alias.
"""
from ._lib import ACT, FaError, lib
from .compute import HipContext, HipTensor, PackedBytes, createContext
from .encoder import FusedEncoder, inferConfig, loadParakeetEncoder, parakeetEncodeBatch, posEncoding, tsub
from .mel import JsPreprocessor, ParakeetMel
from .decoder import TdtDecoder
from . import synth, windowing
from .pipeline import createStitcher, transcribeWindowed
from .streaming import createEncodeStream, disposeEncodeStream, encodeStreamFlush, encodeStreamPush, encodeStreamsPush

__all__ = ["ACT", "FaError", "lib", "HipContext", "HipTensor", "PackedBytes", "createContext", "FusedEncoder", "inferConfig",
           "loadParakeetEncoder", "parakeetEncodeBatch", "posEncoding", "tsub", "synth", "windowing", "JsPreprocessor", "ParakeetMel", "TdtDecoder",
           "createStitcher", "transcribeWindowed",
           "createEncodeStream", "encodeStreamPush", "encodeStreamFlush", "disposeEncodeStream", "encodeStreamsPush"]
