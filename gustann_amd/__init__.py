"""gustann_amd: MI355X-native (gfx950) implementation of GustANN's in-GPU
search path -- PQ LUT build + ADC scan, pivot-graph entry selection, fused
and step-wise beam search with exact rerank -- behind the C ABI of
include/gustann.h (libgustann_hip.so).  See search.GustANN for the facade that
mirrors gustann::GustANN and index for the builders of the reference's file
formats."""
from ._native import (FLOAT, MODE_FUSED, MODE_FUSED_GP, MODE_FUSED_LUT, MODE_STEPWISE, MODE_STEPWISE_PAGED,
                      MODE_STEPWISE_URING,
                      PLACEMENT_HBM,
                      PLACEMENT_HOST_PINNED, UINT8, GannError)
from .search import GustANN, GustANNConfig, GustANNStats, PQSearch

__all__ = ["GustANN", "GustANNConfig", "GustANNStats", "PQSearch", "GannError", "UINT8", "FLOAT",
           "MODE_FUSED", "MODE_FUSED_GP", "MODE_FUSED_LUT", "MODE_STEPWISE", "MODE_STEPWISE_PAGED", "MODE_STEPWISE_URING", "PLACEMENT_HBM", "PLACEMENT_HOST_PINNED"]
