__version__ = "0.1.4+mi355x"
