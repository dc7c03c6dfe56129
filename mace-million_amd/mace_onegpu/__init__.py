"""MI355X-native receiver-chunked three-pass MACE energy + forces.

Module map (mirrors the reference package mace_onegpu, same module paths for the drop-in API):
  mliap_threepass   ThreePassMLIAP: LAMMPS ML-IAP unified plugin, compute_forces(data)
  fused_conv        FusedConvTP: channelwise TP + receiver scatter as an nn.Module
  tp_jit            kernels of path tables without a compiled kernel, built on first use
  receiver_chunk_mace  System (GPU cell-list neighbours), ReceiverChunkMACE (standalone three-pass)
  chunk_graphs      ChunkGraphExec: HIP-graph capture and replay of the passes of full receiver chunks
  md                MDRunner: velocity-Verlet MD with a skin neighbour list (the standalone MD-loop shape)
  make_threepass_model  writes the pickled ThreePassMLIAP model file that pair_style mliap unified loads
  fast_layers       per-chunk layer pipelines on the HIP kernels
  lammps_data       periodic-image ML-IAP data object (one GPU stands in for LAMMPS' ghost exchange)
  model, o3, codegen, systems, _lib   architecture, couplings, kernel generator, inputs, C-ABI binding
"""
__version__ = "0.1.0"
