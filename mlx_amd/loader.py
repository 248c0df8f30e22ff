"""Plugin loader: the reference loader's steps, plus the "hip" name.

Mirrors reference src/plugin_loader.hpp:
  * search paths: defaults /usr/lib/lux-gpu, /usr/local/lib/lux-gpu, with
    LUX_GPU_BACKEND_PATH entries (':'-separated) inserted in front (:112-146),
    plus the directory this package builds the plugin into (the reference's
    "directory of the core library itself", which it leaves unimplemented at
    :144-145);
  * load_backend(name): libluxgpu_backend_<name>.so in each path (:165-182);
  * load_backend_from_path: dlopen(RTLD_NOW | RTLD_LOCAL), dlsym the init
    symbol, call it; init false => registered unavailable; ABI mismatch =>
    message on stderr, library closed, rejected (:184-232);
  * get_best_backend: priority metal, cuda, webgpu (:250-262), extended with
    hip ahead of webgpu (a native GPU backend before the portable one).
and adds what the reference documents but does not implement
(README.md:65): LUX_BACKEND=<name> selects a backend explicitly.  After a
plugin is accepted, the optional quant extension symbol is looked up.
"""
from __future__ import annotations

import ctypes
import os
import sys
from dataclasses import dataclass, field
from typing import Dict, List, Optional

from . import abi

PKG_LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
PRIORITY = ("metal", "cuda", "hip", "webgpu")

try:
    from _ctypes import dlclose as _dlclose
except ImportError:  # pragma: no cover
    _dlclose = None


@dataclass
class LoadedBackend:
    name: str
    path: str
    handle: Optional[ctypes.CDLL]
    desc: abi.BackendDesc = field(default_factory=abi.BackendDesc)
    available: bool = False
    quant: Optional[abi.QuantVtbl] = None

    @property
    def vtbl(self) -> abi.BackendVtbl:
        return self.desc.vtbl.contents


class PluginLoader:
    def __init__(self, env: Optional[Dict[str, str]] = None):
        env = os.environ if env is None else env
        self.search_paths: List[str] = ["/usr/lib/lux-gpu", "/usr/local/lib/lux-gpu", PKG_LIB_DIR]
        # each ':'-separated entry is inserted at the front, as the reference does
        # (so the last entry of the variable ends up first)
        p = env.get("LUX_GPU_BACKEND_PATH", "")
        if p:
            parts = p.split(":")
            for part in parts[:-1]:
                self.search_paths.insert(0, part)
            if parts[-1]:
                self.search_paths.insert(0, parts[-1])
        self.backends: Dict[str, LoadedBackend] = {}
        self.env = env

    # --- reference steps -------------------------------------------------
    def load_backend(self, name: str) -> bool:
        if name in self.backends:
            return self.backends[name].available
        fname = f"libluxgpu_backend_{name}.so"
        for d in self.search_paths:
            if self.load_backend_from_path(os.path.join(d, fname)):
                return True
        return False

    def load_backend_from_path(self, path: str) -> bool:
        if not os.path.exists(path):
            return False
        try:
            handle = ctypes.CDLL(path, mode=os.RTLD_NOW | os.RTLD_LOCAL)
        except OSError:
            return False
        try:
            init = abi.INIT_FN((abi.INIT_SYMBOL.decode(), handle))
        except AttributeError:
            self._close(handle)
            return False
        be = LoadedBackend(name="unknown", path=path, handle=handle)
        if not init(ctypes.byref(be.desc)):
            be.available = False  # backend reports unavailable (e.g. no GPU)
        else:
            if be.desc.abi_version != abi.ABI_VERSION:
                print(f"lux-gpu: backend {path} has ABI version {be.desc.abi_version}, "
                      f"expected {abi.ABI_VERSION}", file=sys.stderr)
                self._close(handle)
                return False
            be.available = True
            be.quant = self._quant_ext(handle)
        be.name = be.desc.backend_name.decode() if be.desc.backend_name else "unknown"
        self.backends[be.name] = be
        return be.available

    def available_backends(self) -> List[str]:
        return ["cpu"] + [n for n, b in self.backends.items() if b.available]

    def get_backend(self, name: str) -> Optional[LoadedBackend]:
        b = self.backends.get(name)
        return b if b is not None and b.available else None

    def get_best_backend(self) -> Optional[LoadedBackend]:
        for n in PRIORITY:
            b = self.get_backend(n)
            if b is not None:
                return b
        return None

    # --- additions -------------------------------------------------------
    def select(self) -> Optional[LoadedBackend]:
        """LUX_BACKEND=<name> loads exactly that backend (None if it is not
        available); unset or "auto" tries every name in priority order."""
        want = self.env.get("LUX_BACKEND", "auto").strip().lower() or "auto"
        if want == "cpu":
            return None  # the core's built-in CPU backend, not a plugin
        if want != "auto":
            return self.get_backend(want) if self.load_backend(want) else None
        for n in PRIORITY:
            self.load_backend(n)
        return self.get_best_backend()

    @staticmethod
    def _quant_ext(handle) -> Optional[abi.QuantVtbl]:
        try:
            qinit = abi.QUANT_INIT_FN((abi.QUANT_INIT_SYMBOL.decode(), handle))
        except AttributeError:
            return None
        p = ctypes.POINTER(abi.QuantVtbl)()
        if not qinit(ctypes.byref(p)) or not p:
            return None
        q = p.contents
        if q.ext_version != abi.QUANT_EXT_VERSION or q.struct_size < ctypes.sizeof(abi.QuantVtbl):
            return None
        return q

    @staticmethod
    def _close(handle) -> None:
        if _dlclose is not None and handle is not None:
            try:
                _dlclose(handle._handle)
            except OSError:
                pass
