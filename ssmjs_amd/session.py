"""MambaSession on the MI355X backend (mirrors src/session/session.ts:206-616).

Same method names, option names, defaults and SessionError codes as the reference. The
methods are synchronous here (the reference's are async; the Node-API binding in
ssmjs_amd/napi keeps the Promise API). Out of this backend's scope, with the reason:
  - BPETokenizer loading (network vocab files): pass `tokenizer` (session.ts:326-334);
  - adapt() (training, MambaTrainer.train): raises after the reference's INPUT_TOO_SHORT check;
  - IndexedDB / download storage (browser APIs): `idbFactory` may be any mutable mapping,
    'fileSystem' reads and writes a file path.
"""
from __future__ import annotations

import time
import urllib.request

from . import _lib
from .errors import SessionError
from .model import HybridMambaModel, MambaTrainer, init_webgpu
from .presets import resolve_model_config
from .streaming import token_stream

RETRY_BASE_DELAY_MS = 500       # session.ts:198
RETRY_BACKOFF_FACTOR = 2        # session.ts:200


def _default_fetch(url: str) -> bytes:
    with urllib.request.urlopen(url, timeout=30) as r:   # noqa: S310 - user-supplied URL
        if getattr(r, "status", 200) >= 400:
            raise OSError(f"HTTP {r.status}")
        return r.read()


class MambaSession:
    def __init__(self, device, tokenizer, model, trainer, name, gpu_mode="webgpu",
                 idb_factory=None):
        self._device = device
        self._tokenizer = tokenizer
        self._model = model
        self._trainer = trainer
        self._name = name
        self._gpuMode = gpu_mode
        self._idb = idb_factory
        self._destroyed = False

    @property
    def gpuMode(self) -> str:
        return self._gpuMode

    # ------------------------------------------------------------------ factory
    @staticmethod
    def create(options: dict, callbacks: dict | None = None) -> "MambaSession":
        """session.ts:243-406."""
        on_progress = (callbacks or {}).get("onProgress")
        name = options.get("name") or "default"
        fetch_retries = options.get("fetchRetries")
        fetch_retries = 2 if fetch_retries is None else fetch_retries
        fetch = options.get("fetch") or _default_fetch
        sleep = options.get("sleep") or time.sleep

        def emit(stage, progress, message):
            if on_progress:
                on_progress({"stage": stage, "progress": progress, "message": message})

        # Step 1 - device
        emit("gpu", 0.0, "Initialising HIP device…")
        gpu_mode = "webgpu"
        adapter = options.get("gpuAdapter")
        if adapter is not None:
            try:
                device = adapter.requestDevice()
            except Exception as err:  # noqa: BLE001 - mirrors the reference's catch-all
                raise SessionError("GPU_UNAVAILABLE",
                                   f"Failed to acquire GPUDevice from provided gpuAdapter: {err}",
                                   err) from err
            emit("gpu", 1.0, "HIP device ready (injected adapter)")
        else:
            try:
                device = init_webgpu({"powerPreference":
                                      options.get("powerPreference") or "high-performance"})["device"]
            except Exception as err:  # noqa: BLE001
                if not options.get("allowCpuFallback"):
                    raise SessionError(
                        "GPU_UNAVAILABLE",
                        f"HIP initialisation failed: {err}. Set allowCpuFallback: true to "
                        "attempt a software (CPU) fallback.", err) from err
                emit("gpu", 0.4, f"HIP unavailable ({err}); attempting CPU software fallback")
                # The MI355X backend has no software adapter; like the reference on Node
                # without one, this is a hard error (session.ts:133,294-300).
                raise SessionError("GPU_UNAVAILABLE",
                                   "No HIP device and no software adapter can be requested.",
                                   err) from err
            emit("gpu", 1.0, "HIP device ready")

        # Step 2 - tokenizer
        emit("tokenizer", 0.0, "Loading tokenizer…")
        tok = options.get("tokenizer")
        if tok is None:
            device.destroy()
            raise SessionError("TOKENIZER_LOAD_FAILED",
                               "Tokenizer failed to load: the BPE vocabulary loader is not part "
                               "of this backend; pass `tokenizer` (a Tokenizer object).")
        emit("tokenizer", 1.0, "Tokenizer ready")

        # Step 3 - model
        emit("model", 0.0, "Building model…")
        vocab = tok.vocabSize if tok.vocabSize > 0 else 1
        config = resolve_model_config(options, vocab)
        try:
            model = HybridMambaModel(device, config, seed=options.get("seed", 0))
        except _lib.SsmError as err:
            device.destroy()
            raise SessionError("UNKNOWN", f"Model construction failed: {err}", err) from err
        trainer = MambaTrainer(model, tok)
        emit("model", 1.0, "Model ready")

        # Step 4 - checkpoint
        url = options.get("checkpointUrl")
        if url is not None:
            emit("weights", 0.0, "Fetching checkpoint…")
            buf, last = None, None
            for attempt in range(fetch_retries + 1):
                try:
                    buf = fetch(url)
                    break
                except Exception as err:  # noqa: BLE001
                    last = err
                    if attempt < fetch_retries:
                        sleep(RETRY_BASE_DELAY_MS * RETRY_BACKOFF_FACTOR ** attempt / 1000.0)
            if buf is None:
                raise SessionError(
                    "CHECKPOINT_FETCH_FAILED",
                    f'Failed to fetch checkpoint from "{url}" after {fetch_retries + 1} '
                    f"attempt(s): {last}", last)
            try:
                model.loadWeights(buf)
            except Exception as err:  # noqa: BLE001
                raise SessionError("CHECKPOINT_INVALID",
                                   f"Checkpoint file is invalid or incompatible: {err}",
                                   err) from err
            emit("weights", 1.0, "Checkpoint loaded")
        return MambaSession(device, tok, model, trainer, name, gpu_mode, options.get("idbFactory"))

    # ------------------------------------------------------------------ generation
    def complete(self, prompt: str, options: dict | None = None, rng=None) -> str:
        """session.ts:410-430."""
        self._assert_not_destroyed()
        o = options or {}
        sampling = {"temperature": o.get("temperature", 0.8), "topK": o.get("topK", 50),
                    "topP": o.get("topP", 0.9)}
        prompt_ids = self._tokenizer.encode(prompt)
        out = self._model.generate(prompt_ids, o.get("maxNewTokens", 200), sampling, rng=rng)
        return self._tokenizer.decode(out[len(prompt_ids):])

    def completeStream(self, prompt: str, options: dict | None = None, rng=None):
        """session.ts:432-454: one decoded piece per generated token."""
        self._assert_not_destroyed()
        o = options or {}
        sampling = {"temperature": o.get("temperature", 0.8), "topK": o.get("topK", 50),
                    "topP": o.get("topP", 0.9)}
        prompt_ids = self._tokenizer.encode(prompt)
        for tid in token_stream(self._model, prompt_ids, o.get("maxNewTokens", 200), sampling,
                                rng=rng):
            yield self._tokenizer.decode([tid])

    def adapt(self, text: str, options: dict | None = None):
        self._assert_not_destroyed()
        if len(self._tokenizer.encode(text)) < 2:
            raise SessionError("INPUT_TOO_SHORT",
                               "The input text encodes to fewer than 2 tokens and cannot be "
                               "used for training.")
        raise SessionError("UNKNOWN", "adapt() (training) is not implemented by the MI355X "
                                      "forward-path backend")

    def evaluate(self, text: str) -> float:
        self._assert_not_destroyed()
        return self._trainer.evaluate(text)

    # ------------------------------------------------------------------ persistence
    def save(self, options: dict | None = None) -> None:
        """session.ts:511-533."""
        self._assert_not_destroyed()
        o = options or {}
        storage = o.get("storage") or "indexedDB"
        key = o.get("key") or self._name
        filename = o.get("filename") or f"{self._name}.bin"
        buf = self._model.exportWeights()
        if storage == "indexedDB":
            if self._idb is None:
                raise SessionError("STORAGE_UNAVAILABLE", "IndexedDB is not available; pass "
                                                          "idbFactory (a mapping)")
            self._idb[key] = buf
        elif storage == "fileSystem":
            with open(filename, "wb") as f:
                f.write(buf)
        elif storage == "download":
            raise SessionError("STORAGE_UNAVAILABLE", "download storage needs a browser")
        else:
            raise SessionError("STORAGE_UNAVAILABLE", f'Unknown storage target: "{storage}"')

    def load(self, options: dict | None = None) -> bool:
        """session.ts:535-585."""
        self._assert_not_destroyed()
        o = options or {}
        storage = o.get("storage") or "indexedDB"
        key = o.get("key") or self._name
        if storage == "indexedDB":
            if self._idb is None:
                raise SessionError("STORAGE_UNAVAILABLE", "IndexedDB is not available; pass "
                                                          "idbFactory (a mapping)")
            buf = self._idb.get(key)
        elif storage == "fileSystem":
            path = o.get("filename") or f"{self._name}.bin"
            try:
                with open(path, "rb") as f:
                    buf = f.read()
            except FileNotFoundError:
                buf = None
        else:
            url = o.get("url")
            if not url:
                raise SessionError("STORAGE_UNAVAILABLE",
                                   'load() with storage other than "indexedDB" or "fileSystem" '
                                   "requires a url option.")
            try:
                buf = (o.get("fetch") or _default_fetch)(url)
            except Exception as err:  # noqa: BLE001
                raise SessionError("CHECKPOINT_FETCH_FAILED",
                                   f'Failed to fetch checkpoint from "{url}": {err}', err) from err
        if buf is None:
            return False
        try:
            self._model.loadWeights(buf)
        except Exception as err:  # noqa: BLE001
            raise SessionError("CHECKPOINT_INVALID",
                               f"Saved checkpoint is invalid or incompatible: {err}",
                               err) from err
        return True

    # ------------------------------------------------------------------ lifecycle
    def destroy(self) -> None:
        if self._destroyed:
            return
        self._destroyed = True
        self._model.destroy()
        self._device.destroy()

    @property
    def internals(self) -> dict:
        return {"device": self._device, "model": self._model, "trainer": self._trainer,
                "tokenizer": self._tokenizer}

    def _assert_not_destroyed(self):
        if self._destroyed:
            raise SessionError("SESSION_DESTROYED",
                               "This MambaSession has been destroyed. Create a new session "
                               "with MambaSession.create().")
