"""What the two HIP backends (FP32- and FP16-accumulated O) share.

Both run the same ``libfa_hip.so`` through the ``hip`` driver and differ only
in the accumulation variant their operator passes to ``fa_fwd``, the way the
reference's two CCE projects share one operator interface
(``backends/cce_fa_nk_nz_vector_fp32_v5_sumpack/backend.py:58-81`` there).
``operator`` opens the built library before any input exists; ``adapt`` maps
the canonical tensors to the operator's positional arguments.
"""


def operator(acc, case, **config):
    """``fa_amd.binding.Operator`` over the built library for variant ``acc``."""
    from fa_amd import build
    from fa_amd.binding import AttentionConfig, Operator

    if not build.LIBRARY.is_file():
        raise FileNotFoundError(f"{build.LIBRARY} is not built (python -m fa_amd.build)")
    return Operator(build.LIBRARY, AttentionConfig(acc=acc, **config))


def adapt(case, canonical):
    return tuple(canonical[name] for name in ("q", "k", "v"))
