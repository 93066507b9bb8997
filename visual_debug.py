"""The ``visual_debug`` module the reference's trainer imports
(manbo/gaussian_trace/render.py:15, model.py:10, legacy.py:5) but does not
ship.  Only its two names are fixed by those call sites: ``VisualDebugHook``,
the type of the trainer's optional ``debug_hook`` argument (model.py:51), and
``emit_visual_debug(hook, stage, payload)`` (render.py:1326, legacy.py:38).
Here a hook is any callable taking ``(stage, payload)``; emitting to ``None``
does nothing, so a trainer built without a hook runs unchanged."""
from __future__ import annotations

from typing import Any, Callable, Mapping, Optional

VisualDebugHook = Callable[[str, Mapping[str, Any]], None]


def emit_visual_debug(hook: Optional[VisualDebugHook], stage: str,
                      payload: Mapping[str, Any]) -> None:
    if hook is None:
        return
    hook(stage, payload)


__all__ = ["VisualDebugHook", "emit_visual_debug"]
