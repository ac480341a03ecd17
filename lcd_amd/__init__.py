"""lcd_amd: an MI355X (gfx950) execution backend for LCD's ``@parallel``.

``from lcd_amd import parallel`` is the drop-in for
``from compiler.decorator import parallel`` of SwiftWare-Lab/lcd.
"""

from lcd_amd.decorator import parallel  # noqa: F401

__all__ = ["parallel"]
