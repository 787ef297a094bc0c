"""ssmjs_amd -- MI355X-native Mamba SSM forward path behind the ssmjs session API.

Public surface (names as in the reference's src/index.ts):
  SSM.create, SSMRuntime, MambaSession, SessionError, SSMError, resolveModelConfig,
  MODEL_PRESETS, tokenStream, sampleToken, HybridMambaModel, MambaTrainer, initWebGPU.
Compute runs in libssm_hip.so (include/ssm_hip.h); importing this package does not load it.
"""
from .errors import SessionError, SSMError
from .model import HipAdapter, HipDevice, HybridMambaModel, MambaTrainer, initWebGPU
from .presets import DEFAULT_PRESET, MODEL_PRESETS, resolveLayerSchedule, resolveModelConfig
from .runtime import SSM, SSMRuntime
from .session import MambaSession
from .streaming import sampleToken, tokenStream
from .tokenizer import ByteTokenizer, Tokenizer

__all__ = ["SSM", "SSMRuntime", "MambaSession", "SessionError", "SSMError",
           "resolveModelConfig", "resolveLayerSchedule", "MODEL_PRESETS", "DEFAULT_PRESET",
           "tokenStream", "sampleToken", "HybridMambaModel", "MambaTrainer", "initWebGPU",
           "HipAdapter", "HipDevice", "Tokenizer", "ByteTokenizer"]
