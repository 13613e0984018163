"""Oracle for the activation-offload path: TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what RyukoMatoiFan/MOSS-Image's
``training/activation_offload.py`` does, so that tests can check the engine against it. It is
the checker, never the thing measured or shipped: only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import, call, link or execute anything here.
The product path (``moss-image_amd/moss_offload``) never imports it and fails loudly when its
HIP library is missing.

Contents
  reference_hooks.py  the reference's hook algorithm (pinned payload + copy + event, restore
                      with empty_strided/copy_/as_strided) and its layout helpers, plus a
                      CPU-payload emulation usable without a GPU
  layout.py           brute-force element-offset enumeration (numpy) that pins the overlap rule
                      and the payload orders (logical order = reference, storage order = engine)
  strided_copy.c      plain-C restatement of the logical-order gather/scatter that
                      ``Tensor.copy_`` performs for a dense payload (reference :75-76, :123-124),
                      with an optional dimension permutation for storage-order payloads
  Makefile / build.py builds strided_copy.c into oracle/_build/liboracle_copy.so

The reference is pure Python; there is no C/C++ reference source to compile, so there is no
``oracle/_ref`` build.
"""
