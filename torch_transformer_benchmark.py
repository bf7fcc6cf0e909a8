#!/usr/bin/env python3
"""Compare numerical accuracy and inference latency between the baseline
Transformer encoder and the MI355X-native candidate.

Correctness rule for every finite output element:
    abs(user - ref) < atol  OR  abs(user - ref) < rtol * abs(ref)

Stable CLI entry point and import-compatible facade of the reference's
torch_transformer_benchmark.py: the allocator environment is configured before
torch is imported (torch_transformer_benchmark.py:18-22 of the reference), then
the harness API is re-exported.  The implementation lives in the
``tiktoktechjam2026track3_amd`` package.

    python torch_transformer_benchmark.py --encoder-configs c2 c3 --json-output result.json
"""

from tiktoktechjam2026track3_amd.runtime_environment import configure_pre_torch_environment

# The allocator reads its configuration while PyTorch is imported: keep this
# before every import below, which import torch.
configure_pre_torch_environment()

from tiktoktechjam2026track3_amd.cases import (  # noqa: E402
    ENCODER_CONFIGS,
    OFFICIAL_TEST_CASES,
    TransformerConfig,
    generate_random_case,
)
from tiktoktechjam2026track3_amd.correctness import (  # noqa: E402
    AccuracyResult,
    AccuracySummary,
    compare_outputs,
    run_accuracy_tests,
)
from tiktoktechjam2026track3_amd.models import (  # noqa: E402
    BaselineSelfAttention,
    BaselineTransformer,
    BaselineTransformerBlock,
    UserOptimizedTransformer,
    copy_model_weights,
)
from tiktoktechjam2026track3_amd.runner import (  # noqa: E402
    config_from_args,
    configure_runtime,
    environment_metadata,
    execution_failed_result,
    is_out_of_memory_error,
    main,
    maybe_compile,
    official_case_result,
    parse_args,
    release_case_memory,
    resolve_device,
    resolve_dtype,
    run_benchmark_case,
    run_encoder_configs,
    run_official_matrix,
    run_single_case,
    settings_metadata,
    validate_args,
    write_json_document,
    write_json_result,
    write_matrix_result,
)
from tiktoktechjam2026track3_amd.profiling import (  # noqa: E402
    PROFILE_CANDIDATE_REPLAYS,
    PROFILE_MAX_CASES,
    PROFILE_MAX_EVENTS,
    PROFILE_WARMUP_REPLAYS,
    profile_candidate,
    summarize_profile_events,
)
from tiktoktechjam2026track3_amd.timing import (  # noqa: E402
    TimingResult,
    benchmark_models,
    benchmark_once,
    percentile,
    warmup_model,
)

__all__ = [
    "ENCODER_CONFIGS", "OFFICIAL_TEST_CASES", "TransformerConfig", "generate_random_case",
    "AccuracyResult", "AccuracySummary", "compare_outputs", "run_accuracy_tests",
    "BaselineSelfAttention", "BaselineTransformer", "BaselineTransformerBlock",
    "UserOptimizedTransformer", "copy_model_weights",
    "config_from_args", "configure_runtime", "environment_metadata", "execution_failed_result",
    "is_out_of_memory_error", "main", "maybe_compile", "official_case_result", "parse_args",
    "release_case_memory", "resolve_device", "resolve_dtype", "run_benchmark_case",
    "run_encoder_configs", "run_official_matrix", "run_single_case", "settings_metadata",
    "validate_args", "write_json_document", "write_json_result", "write_matrix_result",
    "PROFILE_CANDIDATE_REPLAYS", "PROFILE_MAX_CASES", "PROFILE_MAX_EVENTS", "PROFILE_WARMUP_REPLAYS",
    "profile_candidate", "summarize_profile_events",
    "TimingResult", "benchmark_models", "benchmark_once", "percentile", "warmup_model",
]


if __name__ == "__main__":
    raise SystemExit(main())
