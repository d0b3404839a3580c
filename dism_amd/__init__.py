"""dism_amd: MI355X-native (gfx950) flash_dism hard suffix-matching core.

Public API mirrors the reference flash_dism hard path (dism_v3/python/flash_dism/
{hard_forward,hard_backward,summary}.py) on hand-written HIP kernels behind the C ABI of
include/dism_hard.h (libdism_hip.so, loaded with ctypes).
"""
from .hard_backward import backward_hard, backward_hard_recompute
from .hard_forward import forward_hard, hard_dlog_weights, hard_log_weights, hard_readout
from .labels import sign_labels, vocab_argmax_labels, vocab_labels
from .summary import hard_boundary, hard_chunk_scan, summarize_hard
from .core import (dism_core, dism_core_hard, dism_core_hybrid, hard_core, hard_core_backward,
                   voc_dism)
from .varlen import (VarlenLayout, graph_layout_maximum, layout_from_table, make_graph_layout,
                     update_graph_layout)
from .inference import HardDismDecoder, HardDismPrefill, PreparedHardPrefill

__all__ = ["forward_hard", "hard_readout", "hard_log_weights", "hard_dlog_weights",
           "backward_hard", "backward_hard_recompute", "summarize_hard", "hard_chunk_scan",
           "hard_boundary", "sign_labels", "vocab_labels", "vocab_argmax_labels", "dism_core",
           "voc_dism", "dism_core_hybrid",
           "dism_core_hard", "hard_core",
           "hard_core_backward", "VarlenLayout", "make_graph_layout", "update_graph_layout",
           "graph_layout_maximum", "layout_from_table", "HardDismPrefill", "PreparedHardPrefill",
           "HardDismDecoder"]
