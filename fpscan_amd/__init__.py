"""MI355X-native first-order linear-recurrence scan (drop-in for saeeddhqan/fpscan).

Same public names as fpscan/__init__.py:1-3 (``pscan``, ``scan_forward``, ``PScan``), plus
``scan_backward`` (the fused backward, exposed directly) and the channel-last variants for
(batch, seqlen, dim) tensors (``pscan_channel_last``, ``scan_forward_channel_last``,
``scan_backward_channel_last``, ``PScanChannelLast``), and ``dimwise_forward`` (the
reference module's contraction scan, csrc/main.cpp:10) with ``dimwise_groups``, and the
fused gate producer ``pscan_softplus`` (gates exp(-softplus(z) * rate) computed in the
kernels), and ``lookback_overruns`` / ``check_lookback`` (the tiled paths' count of look-back
waits that gave up, whose outputs are NaN).
"""
from .ops import (PScan, PScanChannelLast, PScanSoftplus, check_lookback, dimwise_forward,
                  dimwise_groups, lookback_overruns, pscan, pscan_channel_last, pscan_softplus,
                  scan_backward,
                  scan_backward_channel_last, scan_backward_softplus, scan_forward,
                  scan_forward_channel_last, scan_forward_softplus)

__all__ = ["pscan", "scan_forward", "scan_backward", "PScan", "pscan_channel_last",
           "scan_forward_channel_last", "scan_backward_channel_last", "PScanChannelLast",
           "dimwise_forward", "dimwise_groups", "pscan_softplus", "scan_forward_softplus",
           "scan_backward_softplus", "PScanSoftplus", "lookback_overruns", "check_lookback"]
__version__ = "0.2.0"
