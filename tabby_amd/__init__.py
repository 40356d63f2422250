"""tabby_amd: an MI355X-native (gfx950) implementation of xOAviOx/tabby's token-sampling path.

The sampler itself is the HIP library ``tabby_amd/lib/libtabby_sampler.so`` behind the C ABI
of ``include/tabby_sampler.h``; ``tabby_amd.sampler`` is its Python host side and
``tabby_amd/node`` its Node (N-API) host side.
"""
__version__ = "0.1.0"
