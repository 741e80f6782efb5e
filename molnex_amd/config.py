"""Global dtypes, mirroring molix.config (src/molix/config.py:13-20).

The HIP kernels compute in fp32 (the north-star path); modules bake
``config.ftype`` at construction like the reference (e.g. linear.py:89).
"""

import torch


class _Config:
    ftype: torch.dtype = torch.float32
    itype: torch.dtype = torch.int64
    # True: tensor-product backward walked by sender, without atomics (bitwise
    # reproducible gradients, slower on large graphs)
    deterministic: bool = False
    # True: RadialWeightMLP runs its hidden stack as one fused HIP kernel when its
    # parameters need no gradient (energy + forces); False: always the Sequential
    fused_radial: bool = True
    # True: RadialWeightMLP's last Linear (the per-edge tensor-product weights) runs as the
    # split-fp16 matrix-core kernel molix::edge_weights; False: hipBLASLt fp32 GEMMs
    edge_weights_kernel: bool = True
    # True: an EdgeGraph (the receiver CSR shared by a step's layers) checks once that every
    # edge index lies in [0, num_nodes) -- one host synchronisation per graph; False: trust
    # the indices like the reference's ops (src/molix/F/locality.py:3-5)
    validate_edges: bool = True
    # Where the radial MLP's output layer is frozen and no second derivatives are taken (eval mode),
    # whether the backward forms the output layer's input gradient without writing the per-edge
    # weight gradient (molix::tp_weight_grad_batched with the pairing, molix::radial_tp without it).
    # False (default): never -- on MI355X it breaks even for products of scalar inputs and is slower
    # for inputs with l >= 1 (its per-edge contraction is VALU-bound); None: scalar-input products
    # only (a first interaction layer); True: every product
    fused_weight_grad: bool | None = False
    # True: with the radial MLP run once per undirected pair (paired_radial, eval mode), the tensor
    # product's backward and the output layer's input gradient run as one pass
    # (molix::tp_scatter_backward_gh: the per-edge weight gradient is multiplied on the matrix cores
    # as it is formed, never written) wherever a kernel exists for the product and hidden width.
    # False (default): on MI355X the fused pass is slower than the two kernels it replaces at every
    # measured shape (config 3: 30.3-31.3 ms against 27.4-27.8 ms; the literal config-5 step 29.7-
    # 30.6 ms against 27.6-28.7 ms), since its LDS staging and per-phase barriers cost the receiver
    # walk more occupancy and issue time than the 30.8 GB weight-gradient stream it saves
    tp_bwd_fused: bool = False
    # True: with the radial MLP run once per undirected pair (eval mode), the tensor product's
    # backward runs one path group at a time and each group's columns of the per-edge weight
    # gradient are multiplied into the output layer's input gradient on a second stream while the
    # next group runs (kernels.tp_backward_overlapped).  False (default): the whole backward, then
    # the product; on MI355X the two streams' kernels barely co-reside (the backward's workgroups
    # fill every compute unit's registers), so the overlap saved nothing (config 3 39.5 vs 39.1 ms,
    # literal config 5 29.0 vs 28.6 ms)
    tp_bwd_overlap: bool = False
    # True: where the radial MLP's parameters are frozen and no second derivatives are taken (eval
    # mode), the MLP and its output layer run once per undirected pair of opposite edges whose radial
    # inputs are bit-identical (a neighbor list's pairs), and the tensor product reads each pair's
    # weights for both directions (molix::radial_tp_pairs); graphs without such a pairing run per edge
    paired_radial: bool = True
    # With paired_radial: True -- every new radial-features tensor on a graph (new positions) is
    # checked on the device to keep its pairs bit-identical, with one host synchronisation to read
    # the verdict (a failed check rebuilds the pairing); False -- the pairing found when the graph
    # was first used is trusted for later positions.  That holds whenever the bond vectors of the
    # two directions are exact negations, as molix::bond_vectors makes them from a neighbor list's
    # antisymmetric shifts; it keeps an energy + forces step free of host synchronisation.
    verify_pairs: bool = True


config = _Config()
