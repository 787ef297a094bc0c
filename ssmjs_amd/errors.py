"""Typed errors of the session and runtime layers.

SessionError mirrors src/session/errors.ts:5-24 (same codes, message, optional cause);
SSMError mirrors src/errors/SSMError.ts:9-26.
"""
from __future__ import annotations

SESSION_ERROR_CODES = (
    "GPU_UNAVAILABLE",          # no device / adapter request failed (session.ts:262-316)
    "TOKENIZER_LOAD_FAILED",    # vocab/merges could not be loaded (session.ts:345-351)
    "CHECKPOINT_FETCH_FAILED",  # checkpoint URL failed after retries (session.ts:385-391)
    "CHECKPOINT_INVALID",       # loadWeights threw: bad magic, version or size (session.ts:393-401)
    "INPUT_TOO_SHORT",          # adapt() input shorter than 2 tokens (session.ts:478-484)
    "STORAGE_UNAVAILABLE",      # storage target not available (session.ts:530-531,556-559)
    "SESSION_DESTROYED",        # method called after destroy() (session.ts:608-615)
    "UNKNOWN",
)

SSM_ERROR_CODES = ("RUNTIME_DESTROYED", "BRIDGE_REQUEST_FAILED", "BRIDGE_RESPONSE_INVALID",
                   "MEMORY_UNAVAILABLE", "DISTILL_FAILED", "UNKNOWN")


class SessionError(Exception):
    def __init__(self, code: str, message: str, cause: BaseException | None = None):
        if code not in SESSION_ERROR_CODES:
            raise ValueError(f"unknown SessionErrorCode {code!r}")
        super().__init__(message)
        self.code = code
        self.cause = cause
        self.name = "SessionError"


class SSMError(Exception):
    def __init__(self, code: str, message: str, cause: BaseException | None = None):
        if code not in SSM_ERROR_CODES:
            raise ValueError(f"unknown SSMErrorCode {code!r}")
        super().__init__(message)
        self.code = code
        self.cause = cause
        self.name = "SSMError"
