"""`mtc.nn`: linear layers over packed quadtree weights."""
