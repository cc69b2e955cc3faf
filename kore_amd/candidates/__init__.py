"""Drop-in ``kernel.py`` candidates, one directory per KORE task id."""
