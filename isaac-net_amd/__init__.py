"""isaac_net_amd: a MI355X-native backend for isaac-net's per-control-step network engines.

make_engine("L2", E, R, "cuda", NRConfig(...), backend="hip") returns the NR uplink engine with the reference contract
API (reset / submit / step -> dict / clock / output_schema / counters / state_dict, isaac_net/core/engine.py:319-960);
make_engine("WIFI", ..., NRConfig(wifi=WifiConfig(...))) returns the mean-field 802.11 level
(isaac_net/core/wifi/engine.py:100-403). Both run the hand-written HIP kernels of csrc/ through the C ABI of
include/inet_nr.h and include/inet_wifi.h.
"""
from .config import NRConfig  # noqa: F401
from .phy import PhyTables  # noqa: F401

__version__ = "0.1.0"


def make_engine(*args, **kwargs):
    from .engine import make_engine as _mk
    return _mk(*args, **kwargs)


def __getattr__(name):
    if name in ("HipNREngine", "Requests", "refusals", "HipUnsupported", "set_env_offset"):
        from . import engine
        return getattr(engine, name)
    if name in ("HipWifiEngine", "wifi_refusals"):
        from . import wifi_engine
        return getattr(wifi_engine, name)
    if name == "WifiConfig":
        from .wifi_config import WifiConfig
        return WifiConfig
    raise AttributeError(name)
