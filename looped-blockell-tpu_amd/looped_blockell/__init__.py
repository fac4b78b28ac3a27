"""looped_blockell — MI355X (gfx950) Block-ELL SwiGLU FFN.

A from-scratch HIP implementation of the Block-ELL sparse SwiGLU forward of the
reference's ``looped_blockell`` package, keeping its layer API
(``looped_blockell.layers``) and its ``titan::`` operator schemas
(``looped_blockell.kernels``).  Native code lives in ``liblbk.so`` (kernels +
C ABI, ``include/lbk.h``) and ``_titan_ext.so`` (torch operators).
"""

__version__ = "0.1.0"
