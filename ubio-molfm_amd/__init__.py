"""MI355X-native E2Former-V2 sparse equivariant attention path.

Import name: ``ubio_molfm_amd`` (the directory ``ubio-molfm_amd/`` is loaded
through ``importlib``; see ``load_package`` in the repo-root entry points).

Layout
------
csrc/          HIP kernels for gfx950 and the extern "C" API (libe2v2.so)
_lib.py        ctypes binding of libe2v2.so (fails loudly when it is missing)
build.py       hipcc build of libe2v2.so (in-tree)
ops.py         torch-facing operators and autograd Functions over the C-ABI
sparse_ops.py  the reference's op-level sparse edge functions (first and second order)
neighbors.py   periodic radius graph -> CSR (query rows, key columns); the reference's
               padded-batch construct_radius_neighbor
modules.py     E2former module tree (reference names) on the HIP edge path
model.py       E2FormerBackbone / MolfmAtomic / energy head / forces
calculator.py  E2FormerCalculator-style batched energy+forces entry point
md.py          device-resident velocity-Verlet (NVE) loop
systems.py     seeded synthetic workloads
"""
__version__ = "0.1.0"
