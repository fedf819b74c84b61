"""MI355X (gfx950) batch=1 int4-hier-g32 decode backend for Whetstone.

    whetstone_amd.ffi      ctypes binding of the C ABI (include/whetstone.h)
    whetstone_amd.kernels  safe wrappers with the reference's shape checks
    whetstone_amd.engine   the C++ decode engine (include/whetstone_engine.h)
    whetstone_amd.build    hipcc build of the native libraries
"""
