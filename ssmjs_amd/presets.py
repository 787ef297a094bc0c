"""Model size presets and config resolution (restates src/session/presets.ts:14-121).

Field names follow HybridMambaModelConfig (camelCase), so configs read the same as the
reference's: {vocabSize, dModel, numLayers, dState, dConv, expand, nHeads, nGroups, chunkLen,
mimoGroup, eosId, layers}.
"""
from __future__ import annotations

# src/session/presets.ts:14-19
MODEL_PRESETS = {
    "nano": {"dModel": 128, "numLayers": 4, "dState": 16, "dConv": 4, "expand": 2, "nHeads": 4},
    "small": {"dModel": 256, "numLayers": 6, "dState": 16, "dConv": 4, "expand": 2, "nHeads": 8},
    "medium": {"dModel": 512, "numLayers": 8, "dState": 16, "dConv": 4, "expand": 2, "nHeads": 8},
    "large": {"dModel": 768, "numLayers": 12, "dState": 16, "dConv": 4, "expand": 2, "nHeads": 12},
}

# src/session/presets.ts:21 (the code's default; the doc comment at session.ts:85 says
# 'medium', the code says 'nano', and the code wins)
DEFAULT_PRESET = "nano"


def resolve_layer_schedule(schedule, num_layers: int, default_type: str):
    """src/session/presets.ts:33-55: 'jamba' = every 4th layer attention (index 3, 7, ...),
    rest mamba2; 'zamba' = every 6th layer attention (index 5, 11, ...), rest mamba3; an
    explicit list is returned as given; None repeats default_type."""
    if not schedule:
        return [{"type": default_type} for _ in range(num_layers)]
    if schedule == "jamba":
        return [{"type": "attention" if i % 4 == 3 else "mamba2"} for i in range(num_layers)]
    if schedule == "zamba":
        return [{"type": "attention" if i % 6 == 5 else "mamba3"} for i in range(num_layers)]
    return schedule


def _pick(overrides, preset, key, default):
    v = overrides.get(key)
    if v is None:
        v = preset.get(key)
    return default if v is None else v


def resolve_model_config(options: dict, vocab_size: int) -> dict:
    """src/session/presets.ts:70-121. Resolution order: preset (default 'nano'), then
    modelConfig overrides (only when modelSize == 'custom'), then vocabSize from the
    tokenizer, then mambaVersion as the default layer type, then layerSchedule."""
    size = options.get("modelSize")
    preset_name = DEFAULT_PRESET if size in (None, "custom") else size
    preset = MODEL_PRESETS.get(preset_name, MODEL_PRESETS[DEFAULT_PRESET])
    overrides = options.get("modelConfig") or {} if size == "custom" else {}
    dModel = _pick(overrides, preset, "dModel", 128)
    numLayers = _pick(overrides, preset, "numLayers", 4)
    dState = _pick(overrides, preset, "dState", 16)
    dConv = _pick(overrides, preset, "dConv", 4)
    expand = _pick(overrides, preset, "expand", 2)
    nHeads = _pick(overrides, preset, "nHeads", 4)
    nGroups = _pick(overrides, preset, "nGroups", 1)
    chunkLen = _pick(overrides, preset, "chunkLen", 256)
    mimoGroup = _pick(overrides, preset, "mimoGroup", 1)
    eosId = _pick(overrides, preset, "eosId", -1)
    if dModel % nHeads != 0:
        raise ValueError(
            f"resolveModelConfig: dModel ({dModel}) must be divisible by nHeads ({nHeads}).")
    default_type = options.get("mambaVersion") or "mamba1"
    layers = resolve_layer_schedule(options.get("layerSchedule"), numLayers, default_type)
    cfg = {"vocabSize": vocab_size, "dModel": dModel, "numLayers": numLayers, "dState": dState,
           "dConv": dConv, "expand": expand, "nHeads": nHeads, "nGroups": nGroups,
           "chunkLen": chunkLen, "mimoGroup": mimoGroup, "eosId": eosId, "layers": layers}
    # dt_rank is not a reference config field; the backend uses ceil(dModel / 16).
    for k in ("dtRank", "normEps"):
        if k in overrides:
            cfg[k] = overrides[k]
    return cfg


# camelCase aliases with the reference's names
resolveModelConfig = resolve_model_config
resolveLayerSchedule = resolve_layer_schedule
