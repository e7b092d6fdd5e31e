"""Python front-end of libqorus_hip.so (the MI355X Qorus-IA quantized path).

Thin ctypes bindings over the C-ABI declared in include/qorus.h and
include/qorus_hip.h, plus device-buffer helpers.  There is no CPU fallback:
importing works without a GPU, but every call that needs the device raises
QorusError when libqorus_hip.so is missing or no GPU is usable.
"""
from ._lib import (  # noqa: F401
    LIB_PATH,
    QorusError,
    QTensor,
    DeviceBuffer,
    Stream,
    Event,
    lib,
    check,
    gpu_available,
    q4_tensor,
    f32_tensor,
    Q_OK,
    Q_F32,
    Q_Q4_0,
    ERR,
)
from .model_file import write_qorus_v3, model_layout, QorusHeader  # noqa: F401
from .model import Model, QContext, QLlamaModel, QGenerationState  # noqa: F401
from .tokenizer import Tokenizer, QTokenizer, write_tokenizer, byte_level_vocab  # noqa: F401
from . import synthetic  # noqa: F401
