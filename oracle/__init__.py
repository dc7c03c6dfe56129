"""CPU oracle of the three-pass MACE energy+force path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import this package,
and only as the checker or the timed CPU baseline. The product (``mace-million_amd/``) never imports it.

Contents (each function cites the reference file:line that it restates):
  neighbors.py  numpy restatement of receiver_chunk_mace.System / morton3 / build_neighbors (bit-exact target)
  topology.py   numpy restatement of mliap_threepass._topology / LocalGraph node lists and local indices
  mace_ref.py   fp64 PyTorch-CPU restatement of the model, its full-graph energy/forces, the three-pass
                chunked evaluation (ReceiverChunkMACE.compute) and the fp64-sampled Hermite tables
                (conv_spline.build_tables, spline_radial._sample, spline_w Hermite lookup)
  nlist_c/      plain-C restatement of the cell-list neighbour build (timed CPU baseline of kernel (1))

How each part is pinned is documented in the header of its module and in the tests that pin it.
"""
