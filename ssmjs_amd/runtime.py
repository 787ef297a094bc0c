"""SSMRuntime and the SSM.create namespace (mirror src/runtime/SSMRuntime.ts:78-264 and
src/index.ts:100-108) for the SSM path.

The reference's runtime can route requests to a remote transformer bridge
(src/router/InferenceRouter.ts, src/bridges/); those are network clients with no SSM
arithmetic and are not part of this backend. Without a bridge the reference sends every
request to the session (SSMRuntime.ts:125-150), which is what this runtime does; passing a
bridge raises.
"""
from __future__ import annotations

from types import SimpleNamespace

from .errors import SSMError
from .session import MambaSession


class SSMRuntime:
    def __init__(self, session: MambaSession):
        self._session = session
        self._destroyed = False

    @staticmethod
    def create(opts: dict) -> "SSMRuntime":
        if opts.get("bridge") is not None:
            raise SSMError("UNKNOWN", "transformer bridges and routing are not part of the "
                                      "MI355X SSM backend")
        return SSMRuntime(MambaSession.create(opts["session"], opts.get("callbacks")))

    def generate(self, input: str, opts: dict | None = None, rng=None) -> str:
        self._check_alive()
        o = {k: v for k, v in (opts or {}).items() if k != "bridgeOpts"}
        return self._session.complete(input, o, rng=rng)

    def stream(self, input: str, opts: dict | None = None, rng=None):
        self._check_alive()
        o = {k: v for k, v in (opts or {}).items() if k != "bridgeOpts"}
        yield from self._session.completeStream(input, o, rng=rng)

    def streamHybrid(self, input: str, opts: dict | None = None, rng=None):
        # no bridge: the SSM path (SSMRuntime.ts:170-171)
        yield from self.stream(input, opts, rng)

    def adapt(self, data: str, opts: dict | None = None):
        self._check_alive()
        return self._session.adapt(data, opts)

    def evaluate(self, text: str) -> float:
        self._check_alive()
        return self._session.evaluate(text)

    def save(self, opts: dict | None = None) -> None:
        self._check_alive()
        self._session.save(opts)

    def load(self, opts: dict | None = None) -> bool:
        self._check_alive()
        return self._session.load(opts)

    def getRoutingAuditLog(self) -> list:
        return []

    def getDistillationLog(self) -> list:
        return []

    @property
    def bridge(self):
        return None

    @property
    def destroyed(self) -> bool:
        return self._destroyed

    @property
    def internals(self) -> dict:
        return self._session.internals

    def destroy(self) -> None:
        self._session.destroy()
        self._destroyed = True

    def _check_alive(self):
        if self._destroyed:
            raise SSMError("RUNTIME_DESTROYED", "SSMRuntime has been destroyed.")


SSM = SimpleNamespace(create=SSMRuntime.create)
