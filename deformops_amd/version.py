"""Version of the MI355X MSDA build."""

__version__ = "0.1.0"
