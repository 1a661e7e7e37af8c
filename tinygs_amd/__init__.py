"""tinygs_amd: MI355X-native FastGS training path (placeholder, filled in below)."""
from . import image, scenes  # noqa: F401
