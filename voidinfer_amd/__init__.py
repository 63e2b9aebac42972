"""voidinfer_amd — MI355X (gfx950) token sampling and speculative-decode acceptance.

The compute path is ``libvoidinfer_sampling.so`` (hand-written HIP kernels behind
the C ABI in ``include/voidinfer_sampling.h``).  Importing this package loads
that library and fails with ImportError if it has not been built; nothing here
falls back to a CPU implementation.
"""
from ._abi import (ABSENT_OCCURRENCE, BF16, F16, F32, FLAG_BAD_HISTORY, FLAG_EMPTY, FLAG_ERROR,  # noqa: F401
                   FLAG_NO_RESIDUAL, FLAG_NONFINITE, FLAG_ZERO_Q, GREEDY_ROW, LIB_PATH, ROUTE_ALL, ROUTE_FULL,
                   ROUTE_TOPK, ROW_PARAMS,
                   SAMPLE_STATS, VERIFY_GREEDY, VERIFY_SAMPLED, VERIFY_SAMPLED_TOPK, DRAFT_SAMPLING, DeviceSampling, VIError, load)

load()

from .ops import (PacketTransport, PenaltyState, draft_choice, greedy_packet, params_array, presence_record, presence_reset,  # noqa: E402,F401
                  presence_truncate, probe_copy, probe_read, route_mask, row_scores, sample_rows, sample_rows_state,
                  sampled_packet, sampled_scores, selector_chain, stats_numpy,
                  to_device_bytes, topk_rows,
                  verification_tree, verify_rows, workspace)
