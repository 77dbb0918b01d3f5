"""ComfyUI-INT4-ConvRot for AMD MI355X (gfx950 / CDNA4).

The W4A4 ConvRot linear path of the RDNA4 node, rebuilt for gfx950: the
``Int4ConvRotOps`` Linear replacement (``int4_ops``) over the ``_int4``
backend, whose rotate+quantize and W4A4 GEMM run as hand-written HIP kernels
(``csrc/``) behind a C-ABI library.

The ComfyUI node classes (loader / save / pre-LoRA UI) are not part of this
package; the reference's nodes construct ``Int4ConvRotOps`` and call the
``_int4`` API, both of which are provided here with the same names.
"""
NODE_CLASS_MAPPINGS = {}
NODE_DISPLAY_NAME_MAPPINGS = {}

__all__ = ["NODE_CLASS_MAPPINGS", "NODE_DISPLAY_NAME_MAPPINGS"]
