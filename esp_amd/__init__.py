"""MI355X-native llama-family decoder forward behind esp's model-execution API.

The compute path is the HIP library esp_amd/libesp_hip.so (C ABI in
include/esp_hip.h); this package is the host-side mirror of the reference's
decoder interface (config parsing, model/KV handles, the generation loop and
the sampler) driving that library through ctypes.
"""
from .errors import (Backend, InferError, Interrupted, InvalidConfig, InvalidRequest,  # noqa: F401
                     InvalidWeights, ModelNotLoaded, PromptTooLong, StageUnavailable, Unsupported)
from .config import DecoderConfig, MoeConfig, RopeScaling  # noqa: F401
from .model import DecoderModel, KvCache  # noqa: F401
from .generate import (TokenPicker, generate_constrained, generate_ids,  # noqa: F401
                       generate_ids_with)
from .sample import Sampler  # noqa: F401
from .provider import (DecoderProvider, GenerationCheckpoint, GenerationRequest,  # noqa: F401
                       ScoreHealth)
from .constraint import Constraint, Vocabulary  # noqa: F401
from .streaming import (ArtifactSource, FnSource, LayerSource, StreamingOptions,  # noqa: F401
                        cache_verified_layers, split_checkpoint, with_expert_reader)
