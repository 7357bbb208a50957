"""Kernel definitions of the quantized mul_mat path.

Each object stands where the reference has an ``@weft.kernel`` DSL function
(examples/kernels/...): it carries the symbol name, the Python signature (the
View parameters in order) and the declared alias groups, which is all the
runtime needs (python/weft/api/definitions.py:36-85).  The body is the
hand-written gfx950 code behind the same symbol in libweft_hip, so there is
no DSL to lower.  Calling a definition directly raises LanguageUseError, as
the reference does.
"""
from __future__ import annotations

import inspect
from collections.abc import Mapping

from .diagnostics import DefinitionError, LanguageUseError


class KernelDefinition:
    def __init__(self, name: str, parameters: tuple[str, ...], source: str,
                 alias_groups: Mapping[str, str] | None = None,
                 source_bindings: tuple[str, ...] = ()) -> None:
        groups = dict(alias_groups or {})
        if any(not isinstance(k, str) or not k or not isinstance(v, str) or not v
               for k, v in groups.items()):
            raise DefinitionError("kernel alias_groups maps parameter names to non-empty group names")
        unknown = set(groups).difference(parameters)
        if unknown:
            raise DefinitionError(f"kernel alias_groups names unknown parameters: {', '.join(sorted(unknown))}")
        self.__name__ = name
        self.__qualname__ = name
        self.parameters = tuple(parameters)
        self.alias_groups = groups
        self.source = source
        # names of the reference kernel's ``wl.auto`` extents: each needs one
        # concrete ``CompileOptions.meta`` binding at compile time
        self.source_bindings = tuple(sorted(source_bindings))

    @property
    def signature(self) -> inspect.Signature:
        return inspect.Signature([inspect.Parameter(p, inspect.Parameter.POSITIONAL_OR_KEYWORD)
                                  for p in self.parameters])

    def __call__(self, *args, **kwargs):
        raise LanguageUseError(
            f"kernel {self.__name__} is a definition; use weft_amd.runtime.jit or compile to execute it")

    def __repr__(self) -> str:
        return f"<weft_amd kernel {self.__name__}>"


_MM = ("W", "X", "Xq", "Y")
_MM_IQ2 = ("W", "X", "Xq", "grid", "signs", "Y")
_MM_MX = ("W", "X", "Xq", "codebook", "scale", "Y")
_DECODE_GROUPS = {"Xq": "workspace", "Y": "output"}

# wl.auto extents of the tiled prefill kernels (mul_mat/q4_0.py:17-22,
# q4_k_staged.py:20-24, iq2_xxs_staged.py:43-48 and :80-83, mxfp4.py:21-25,
# q6_k.py:17-21, q5_k.py:17-22, nvfp4.py:21-26)
_AUTO = {
    "production_mul_mat_q4_0": ("MC", "MR", "NC", "NR"),
    "production_mul_mat_q4_k_staged": ("KC", "MC", "MR", "NC"),
    "production_mul_mat_iq2_xxs_staged": ("KC", "MC", "MR", "NC", "NR"),
    "production_mul_mat_mxfp4": ("MC", "MR", "NC", "NR"),
    "production_mul_mat_q6_k": ("MC", "MR", "NC", "NR"),
    "production_mul_mat_q5_k": ("MC", "MR", "NC", "NR"),
    "production_mul_mat_nvfp4": ("MC", "MR", "NC", "NR"),
    "production_mul_mat_q4_1": ("MC", "MR", "NC", "NR"),
    "production_mul_mat_iq2_xs": ("NR",),
    "production_mul_mat_iq2_xs_staged": ("KC", "MC", "MR", "NC", "NR"),
}

# (symbol, parameters, reference source, alias groups)
_DEFS = [
    ("row_dequantize_q4_0", ("W", "Y"), "examples/kernels/dequantize/q4_0.py:9-13", None),
    ("row_dequantize_q4_k", ("W", "Y"), "examples/kernels/dequantize/q4_k.py:9-20", {"Y": "output"}),
    ("row_dequantize_iq2_xxs", ("W", "grid", "signs", "Y"), "examples/kernels/dequantize/iq2_xxs.py:9-53",
     {"Y": "output"}),
    ("row_dequantize_mxfp4", ("W", "codebook", "scale", "Y"), "examples/kernels/dequantize/mxfp4.py:9-20", None),
    ("q8_0_quantize", ("X", "Y"), "examples/kernels/quantize/q8_0.py:26-28", None),
    ("q8_K_quantize", ("X", "Y"), "examples/kernels/quantize/q8_k.py:38-40", None),
    ("quantized_vec_dot_q4_0_q8_0", ("W", "X", "Y"), "examples/kernels/vec_dot/q4_0_q8_0.py:19-23", None),
    ("quantized_vec_dot_q4_k_q8_k", ("W", "X", "Y"), "examples/kernels/vec_dot/q4_k_q8_k.py:32-36", None),
    ("quantized_vec_dot_iq2_xxs_q8_k", ("W", "X", "grid", "signs", "Y"),
     "examples/kernels/vec_dot/iq2_xxs_q8_k.py:46-54", None),
    ("quantized_vec_dot_mxfp4_q8_0", ("W", "X", "codebook", "scale", "Y"),
     "examples/kernels/vec_dot/mxfp4_q8_0.py:25-33", None),
    ("production_mul_mat_q4_0", _MM, "examples/kernels/mul_mat/q4_0.py:9-30", None),
    ("production_mul_mat_q4_0_decode", _MM, "examples/kernels/mul_mat/q4_0_decode.py:10-20", None),
    ("production_mul_mat_q4_k", _MM, "examples/kernels/mul_mat/q4_k.py:10-20", None),
    ("production_mul_mat_q4_k_decode", _MM, "examples/kernels/mul_mat/q4_k_decode.py:10-20", _DECODE_GROUPS),
    ("production_mul_mat_q4_k_staged", _MM, "examples/kernels/mul_mat/q4_k_staged.py:9-37", None),
    ("production_mul_mat_iq2_xxs", _MM_IQ2, "examples/kernels/mul_mat/iq2_xxs.py:10-23", None),
    ("production_mul_mat_iq2_xxs_decode", _MM_IQ2, "examples/kernels/mul_mat/iq2_xxs_decode.py:10-23",
     _DECODE_GROUPS),
    ("production_mul_mat_iq2_xxs_staged", _MM_IQ2, "examples/kernels/mul_mat/iq2_xxs_staged.py:86-97",
     _DECODE_GROUPS),
    ("production_mul_mat_mxfp4", _MM_MX, "examples/kernels/mul_mat/mxfp4.py:10-35", None),
    ("production_mul_mat_mxfp4_decode", _MM_MX, "examples/kernels/mul_mat/mxfp4_decode.py:10-23",
     _DECODE_GROUPS),
    ("row_dequantize_q6_k", ("W", "Y"), "examples/kernels/dequantize/q6_k.py:8-15", None),
    ("quantized_vec_dot_q6_k_q8_k", ("W", "X", "Y"), "examples/kernels/vec_dot/q6_k_q8_k.py:39-44", None),
    ("production_mul_mat_q6_k", _MM, "examples/kernels/mul_mat/q6_k.py:9-37", _DECODE_GROUPS),
    ("production_mul_mat_q6_k_decode", _MM, "examples/kernels/mul_mat/q6_k_decode.py:10-20", None),
    ("row_dequantize_q5_k", ("W", "Y"), "examples/kernels/dequantize/q5_k.py:9-15", {"Y": "output"}),
    ("quantized_vec_dot_q5_k_q8_k", ("W", "X", "Y"), "examples/kernels/vec_dot/q5_k_q8_k.py:34-38", None),
    ("production_mul_mat_q5_k", _MM, "examples/kernels/mul_mat/q5_k.py:9-37", None),
    ("production_mul_mat_q5_k_decode", _MM, "examples/kernels/mul_mat/q5_k_decode.py:10-20", None),
    ("row_dequantize_nvfp4", ("W", "codebook", "scale", "Y"), "examples/kernels/dequantize/nvfp4.py:9-24", None),
    ("quantized_vec_dot_nvfp4_q8_0", ("W", "X", "codebook", "scale", "Y"),
     "examples/kernels/vec_dot/nvfp4_q8_0.py:29-38", None),
    ("production_mul_mat_nvfp4", _MM_MX, "examples/kernels/mul_mat/nvfp4.py:10-43", None),
    ("production_mul_mat_nvfp4_decode", _MM_MX, "examples/kernels/mul_mat/nvfp4_decode.py:10-23", None),
    ("production_mul_mat_q4_k_persistent", _MM, "examples/kernels/mul_mat/q4_k_persistent.py:10-31", None),
    ("row_dequantize_q4_1", ("W", "Y"), "examples/kernels/dequantize/q4_1.py:9-13", None),
    ("row_dequantize_iq2_xs", ("W", "grid", "signs", "Y"), "examples/kernels/dequantize/iq2_xs.py:9-75", None),
    ("q8_1_quantize", ("X", "Y"), "examples/kernels/quantize/q8_1.py:28-30", None),
    ("quantized_vec_dot_q4_1_q8_1", ("W", "X", "Y"), "examples/kernels/vec_dot/q4_1_q8_1.py:8-29", None),
    ("quantized_vec_dot_iq2_xs_q8_k", ("W", "X", "grid", "signs", "Y"),
     "examples/kernels/vec_dot/iq2_xs_q8_k.py:9-45", None),
    ("production_mul_mat_q4_1", _MM, "examples/kernels/mul_mat/q4_1.py:9-30", _DECODE_GROUPS),
    ("production_mul_mat_q4_1_decode", _MM, "examples/kernels/mul_mat/q4_1_decode.py:10-20", _DECODE_GROUPS),
    ("production_mul_mat_iq2_xs", _MM_IQ2, "examples/kernels/mul_mat/iq2_xs.py:26-56", _DECODE_GROUPS),
    ("production_mul_mat_iq2_xs_staged", _MM_IQ2, "examples/kernels/mul_mat/iq2_xs_staged.py:29-75", None),
    ("q4_k_q8_k_gemv", ("W", "X", "Y"), "examples/kernels/gemv/q4_k.py:8-26", None),
    ("q4_k_q8_k_gemv_groups4", ("W", "X", "Y"), "examples/kernels/gemv/q4_k_groups4.py:8-26", None),
    ("q4_k_q8_k_gemv_contract", ("W", "X", "Y"), "examples/kernels/gemv/q4_k_contract.py:8-26", None),
]

DEFINITIONS: dict[str, KernelDefinition] = {}
for _name, _params, _src, _groups in _DEFS:
    DEFINITIONS[_name] = KernelDefinition(_name, _params, _src, _groups, _AUTO.get(_name, ()))
    globals()[_name] = DEFINITIONS[_name]

__all__ = ["KernelDefinition", "DEFINITIONS", *DEFINITIONS]
