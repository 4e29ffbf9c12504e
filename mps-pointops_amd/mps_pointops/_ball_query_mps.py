"""The reference's import path for the dense ball query
(``mps_pointops._ball_query_mps``); on this build it is served by the ROCm
implementation in ``mps_pointops._ball_query``."""

from ._ball_query import (  # noqa: F401
    BallQueryResult,
    _BallQuery,
    _checked_radius_and_k,
    _lengths_or_full,
    ball_query,
)
