"""gfx950 (MI355X) implementation of the Flash-Next quantized MoE expert path.

Drop-in for the reference's ``models/flashnext`` expert path:

* ``hip_runtime``  ``HipMoEExecutor`` -- the ``MetalMoEExecutor`` surface
* ``ops``          ``quantized_matmul`` / ``gather_qmm`` / ``dequantize``
* ``router``       softmax / top-k / renorm / slot words on the device
* ``moe_block``    the ``_moe_call`` composition (router + experts + shared)
* ``grouped``      prefill / verify grouped path (sorted rows, MFMA GEMMs)
* ``pool``         HBM-resident slot pool with LRU and pinned-host refill
* ``layout``       the expert record layout
* ``_lib``         ctypes binding of ``libmqmoe.so`` (``include/mqmoe.h``)

Submodules are imported on demand so that ``_lib`` and ``layout`` load
without torch.
"""

__version__ = "0.1.0"
