"""Which kernel family serves a GEMM call, as the library dispatches it (``gemm_impl`` in
``litevllm_amd/csrc/awq_capi.hip``): the decode kernels multiply the unrounded weights
(q - z) * s, the prefill kernels the weights rounded once to the activation dtype, so a test's
exact reference takes the matching weights."""


def decode_serves(M: int, N: int, G: int) -> bool:
    """M <= 32 on the decode kernels, and 32-row chunks of them up to M = 64, for group sizes
    32, 64 and 128 (N does not enter the rule)."""
    return int(G) in (32, 64, 128) and M <= 64
