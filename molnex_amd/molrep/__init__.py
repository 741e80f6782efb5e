"""molrep (hot-path subset) on the HIP kernels: embeddings, interaction blocks, readout."""
