"""MI355X (gfx950) implementation of the Wan2.2-A14B DiT-block hot path.

Drop-ins for the reecedantin/vllm-omni-neuron op boundary of the Wan2.2 transformer block
(``adaln_modulate``, ``row_quantize_packed``, ``row_mx_qkv_proj``, ``row_mx_mlp``, ``row_mx_o_proj``,
``wan_cp_self_attention``/``_nki_attend``, ``ring_attention_const_max_fwd``), each backed by
hand-written HIP kernels in ``libwanmi.so`` and called through its C ABI (``include/wanmi.h``).

The directory name contains dashes, so it is imported under the module name
``vllm_omni_neuron_amd`` by :func:`__graft_entry__.load_package`.
"""

from . import _lib  # noqa: F401
from .adaln_kernels import AdaLNQuantKernelArgs, adaln_modulate, adaln_quant_kernel  # noqa: F401
from .common_types import DtypeMode, MXTensor, NormType, QKNormConfig, QKVOutputLayout, QuantizationType  # noqa: F401
from .row_mx_kernels import (  # noqa: F401
    MXWeight,
    mxfp8_linear,
    mxfp8_qkv_linear,
    packed_weight_to_mx,
    quantize_weight_mx,
    row_mx_mlp,
    row_quantize_packed,
)
from . import rope  # noqa: F401
from .rope import WanRotaryPosEmbed, rope_tables  # noqa: F401
from . import attention_ops  # noqa: F401
from .attention_ops import (  # noqa: F401
    _nki_attend,
    ring_attention_const_max_fwd,
    row_mx_o_proj,
    row_mx_qkv_proj,
    wan_cp_self_attention,
)
attention_ops.register_torch_ops()
from . import block  # noqa: F401
from . import comfy_fp8_checkpoint  # noqa: F401
from . import kernels  # noqa: F401
from . import row_block  # noqa: F401
