"""Reference-shaped decode API (afterimage.runtime's codec modules) on gfx950."""
